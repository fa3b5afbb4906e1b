// mmq_skinny.hip -- int8-MFMA GEMM for decode batches (3 <= M <= 32) on
// gfx950, where the weight stream still bounds the time but the v_dot4
// GEMV would spend more VALU time than the weights take to arrive.
//
// Replaces the reference's MMQ kernels for 9 <= M <= 64
// (runtime/backends/cuda/native/kernels/mmq.cuh:41-835; dispatch
// fused_quant_gemm.cu:1705-1738) and the M = 3..8 MMVQ columns
// (kernels/mmvq.cuh:49-158), with the same arithmetic: an exact integer dot
// per 32-value block (two 16-value halves for Q6_K), then fp32 scaling by
// the weight and the Q8_1 activation block scales; the Q4_K min term uses
// the Q8_1 s field (mmvq.cuh:115-125, 467-471, 886-889).
//
// Mapping: v_mfma_i32_16x16x32_i8 with rows = batch rows m (A = Q8_1 codes)
// and columns = weight rows n (B = unpacked weight codes).  Lane l supplies
// A row l % 16 and B column l % 16 for the 8-value K chunk l / 16, and
// receives column n = l % 16 and rows 4*(l/16) + i, i < 4, of the result.
//  * A workgroup is 4 waves; each wave owns one n-tile of 16 weight rows and
//    all MT m-tiles of 16 batch rows.  The workgroup walks a range of
//    super-blocks (256 values of K).  Per super-block the four waves stage
//    the batch rows' Q8_1 blocks once in LDS (shared) and each wave stages
//    its own 16 weight rows (raw bytes: 144 B Q4_K, 210 B Q6_K, 8 x 34 B
//    Q8_0) -- 16-byte buffer loads whose lanes cover contiguous memory --
//    then reads the MFMA operands from LDS.  The next super-block's loads
//    are issued before the current one is computed.
//  * Small N cannot fill 256 CUs with 16-row tiles, so the super-blocks are
//    split across gridDim.y workgroups whose fp32 partial sums are added to
//    Y with atomics (Y is zeroed first for the store/bias modes).  Then the
//    summation order, hence the last bits of y, can vary between runs, as
//    in the reference's atomic fp32 accumulate kernels (mmvq.cuh:280-401).
//    fp16 outputs never split.
//  * Scaling: Q4_K and Q6_K sub-block scales are integers, so each block's
//    int32 result is multiplied by its scale in the integer pipe (24-bit
//    multiply) and the fp32 sum is taken in units of the super-block d (one
//    multiply by d per super-block).  The Q4_K min term sum_b (dmin*m_b)*s_b
//    is a small fp32 GEMM done on the matrix cores (v_mfma_f32_16x16x4f32).
#include "ifx_common.h"

#include <stdlib.h>

namespace ifx {

namespace {

constexpr int kWaves = 4;

__device__ __forceinline__ i32x4 mfma16x16x32(int64_t a, int64_t b) {
  const i32x4 z = {0, 0, 0, 0};
  return __builtin_amdgcn_mfma_i32_16x16x32_i8(a, b, z, 0, 0, 0);
}

// Q6_K code bytes v in [0, 63] -> int8 (v - 32), four per dword, no carries.
__device__ __forceinline__ uint32_t q6_minus32(uint32_t v) {
  uint32_t x = v ^ 0x20202020u;
  const uint32_t t = x & 0x20202020u;
  return x | (t << 1) | (t << 2);
}

__device__ __forceinline__ int64_t pack64(uint32_t lo, uint32_t hi) {
  return static_cast<int64_t>(static_cast<uint64_t>(lo) | (static_cast<uint64_t>(hi) << 32));
}

template <int QT>
struct WFmt;
template <>
struct WFmt<kTypeQ4_K> {  // one super-block of a row: 144 raw bytes
  static constexpr int kSbBytes = 144, kPitch = 144, kChunks = 9;
};
template <>
struct WFmt<kTypeQ6_K> {  // 210 raw bytes; the 14th chunk carries only d
  static constexpr int kSbBytes = 210, kPitch = 224, kChunks = 14;
};
template <>
struct WFmt<kTypeQ8_0> {  // 8 blocks x 34 bytes
  static constexpr int kSbBytes = 272, kPitch = 272, kChunks = 17;
};

constexpr int kApitch = 288;  // 8 Q8_1 blocks x 36 bytes per batch row
constexpr int kAChunks = 18;

template <int QT, int MT>
struct Stage {
  static constexpr int kABytes = 16 * MT * kApitch;              // shared
  static constexpr int kWBytes = 16 * WFmt<QT>::kPitch;          // per wave
  static constexpr int kBytes = kABytes + kWaves * kWBytes;
  static constexpr int kWChunks = 16 * WFmt<QT>::kChunks;        // per wave
  static constexpr int kAChunksAll = 16 * MT * kAChunks;         // per workgroup
  static constexpr int kWPerLane = (kWChunks + 63) / 64;
  static constexpr int kAPerThread = (kAChunksAll + 64 * kWaves - 1) / (64 * kWaves);
};

// One super-block's chunks held by this lane, and their loop-invariant
// byte offsets (super-block sb adds sb * bytes-per-super-block).
template <int QT, int MT>
struct StageRegs {
  u32x4 w[Stage<QT, MT>::kWPerLane];
  u32x4 a[Stage<QT, MT>::kAPerThread];
};
template <int QT, int MT>
struct StageOffsets {
  uint32_t w[Stage<QT, MT>::kWPerLane];
  int32_t a[Stage<QT, MT>::kAPerThread];  // -1: batch row past M (zero)
};

template <int QT, int MT>
__device__ __forceinline__ void stage_offsets(StageOffsets<QT, MT> &so, int n0, int N, int M,
                                              uint32_t w_row, uint32_t a_row, int lane, int tid) {
  using S = Stage<QT, MT>;
  using F = WFmt<QT>;
#pragma unroll
  for (int i = 0; i < S::kWPerLane; ++i) {
    const int c = min(lane + 64 * i, S::kWChunks - 1);
    const int r = c / F::kChunks, part = c - r * F::kChunks;
    so.w[i] = static_cast<uint32_t>(min(n0 + r, N - 1)) * w_row + part * 16;
  }
#pragma unroll
  for (int i = 0; i < S::kAPerThread; ++i) {
    const int c = min(tid + 64 * kWaves * i, S::kAChunksAll - 1);
    const int r = c / kAChunks, part = c - r * kAChunks;
    so.a[i] = (r < M) ? static_cast<int32_t>(r * a_row + part * 16) : -1;
  }
}

template <int QT, int MT>
__device__ __forceinline__ void load_stage(StageRegs<QT, MT> &rg, const StageOffsets<QT, MT> &so,
                                           rsrc_t Wr, rsrc_t Ar, int sb, int lane, int tid) {
  using S = Stage<QT, MT>;
  using F = WFmt<QT>;
  const uint32_t wsb = sb * F::kSbBytes;
  const uint32_t asb = sb * kApitch;
#pragma unroll
  for (int i = 0; i < S::kWPerLane; ++i) {
    const int c = lane + 64 * i;
    rg.w[i] = u32x4{0, 0, 0, 0};
    if (S::kWChunks % 64 == 0 || i + 1 < S::kWPerLane || c < S::kWChunks) {
      if (QT == kTypeQ6_K && (c % F::kChunks) == 13) rg.w[i].x = bload<uint16_t>(Wr, so.w[i], wsb);
      else rg.w[i] = bload<u32x4>(Wr, so.w[i], wsb);
    }
  }
#pragma unroll
  for (int i = 0; i < S::kAPerThread; ++i) {
    const int c = tid + 64 * kWaves * i;
    rg.a[i] = u32x4{0, 0, 0, 0};
    if ((S::kAChunksAll % (64 * kWaves) == 0 || i + 1 < S::kAPerThread || c < S::kAChunksAll) &&
        so.a[i] >= 0)
      rg.a[i] = bload<u32x4>(Ar, static_cast<uint32_t>(so.a[i]), asb);
  }
}

template <int QT, int MT>
__device__ __forceinline__ void store_stage(uint8_t *as, uint8_t *ws, const StageRegs<QT, MT> &rg,
                                            int lane, int tid) {
  using S = Stage<QT, MT>;
  using F = WFmt<QT>;
#pragma unroll
  for (int i = 0; i < S::kWPerLane; ++i) {
    const int c = lane + 64 * i;
    if (S::kWChunks % 64 == 0 || i + 1 < S::kWPerLane || c < S::kWChunks) {
      const int r = c / F::kChunks, part = c - r * F::kChunks;
      *reinterpret_cast<u32x4 *>(ws + r * F::kPitch + part * 16) = rg.w[i];
    }
  }
#pragma unroll
  for (int i = 0; i < S::kAPerThread; ++i) {
    const int c = tid + 64 * kWaves * i;
    if (S::kAChunksAll % (64 * kWaves) == 0 || i + 1 < S::kAPerThread || c < S::kAChunksAll)
      *reinterpret_cast<u32x4 *>(as + c * 16) = rg.a[i];
  }
}

}  // namespace

// Up to three projections over the same activations (grouped launches):
// workgroups [seg[i].blk_begin, seg[i + 1].blk_begin) belong to projection i.
struct SkSeg {
  const uint8_t *W;
  void *Y;
  const void *bias;
  int N;
  int blk_begin;
};
struct SkArgs {
  SkSeg seg[3];
  int nseg;
  const uint8_t *A;
  int M, K, mode, sb_per;
};

// Zeroes up to three fp32 outputs (the split-K kernels add into them);
// blockIdx.y selects the output.  Four floats per thread, one 16-byte store
// where the output is 16-byte aligned.
__global__ __launch_bounds__(256) void k_fill_zero(const FillArgs f) {
  float *__restrict__ y = f.y[blockIdx.y];
  const int64_t n = f.n[blockIdx.y];
  const int64_t i = (static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x) * 4;
  if (i >= n) return;
  if ((reinterpret_cast<uintptr_t>(y) & 15) == 0 && i + 4 <= n) {
    *reinterpret_cast<f32x4 *>(y + i) = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  } else {
    for (int64_t j = i; j < n && j < i + 4; ++j) y[j] = 0.0f;
  }
}

hipError_t launch_fill_zero(const FillArgs &f, int nseg, hipStream_t s) {
  int64_t nmax = 0;
  for (int i = 0; i < nseg; ++i) nmax = max(nmax, f.n[i]);
  if (nmax == 0) return hipSuccess;
  IFX_LAUNCH0(k_fill_zero, dim3(static_cast<unsigned>((nmax + 1023) / 1024), nseg),
                     dim3(256), 0, s, f);
  return peek_error();  // left set for the caller's hipGetLastError
}

// grid: x = row groups of 64 (all projections), y = super-block splits.
// Pipeline: the LDS stage is double-buffered and two super-blocks are in
// flight in registers, so a step has one barrier and its loads were issued
// two steps earlier.
template <int QT, int MT, bool F16OUT, bool ATOMIC>
__global__ __launch_bounds__(64 * kWaves, 2) void k_mmq_skinny(const SkArgs args) {
  using S = Stage<QT, MT>;
  using F = WFmt<QT>;
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const int bx = blockIdx.x;
  const int si = (args.nseg > 2 && bx >= args.seg[2].blk_begin) ? 2
                 : (args.nseg > 1 && bx >= args.seg[1].blk_begin) ? 1 : 0;
  const SkSeg &sg = args.seg[si];
  const uint8_t *__restrict__ W = sg.W;
  const uint8_t *__restrict__ A = args.A;
  void *__restrict__ Y = sg.Y;
  const void *__restrict__ bias = sg.bias;
  const int N = sg.N, M = args.M, K = args.K, mode = args.mode, sb_per = args.sb_per;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform
  const int l16 = lane & 15, kq = lane >> 4;
  const int n0 = ((bx - sg.blk_begin) * kWaves + wave) * 16;
  const int nblk = K >> 5;  // Q8_1 blocks per activation row
  const int nsb = K >> 8;   // super-blocks of 256 values
  const int sb0 = blockIdx.y * sb_per;
  const int sb1 = min(nsb, sb0 + sb_per);
  // two stage buffers: shared batch rows, then each wave's weight rows
  uint8_t *const buf[2] = {smem, smem + S::kBytes};

  const uint32_t w_row = static_cast<uint32_t>(QT == kTypeQ8_0 ? nblk * kQ8_0Bytes : nsb * F::kSbBytes);
  const uint32_t a_row = static_cast<uint32_t>(nblk) * kQ8_1Bytes;
  const rsrc_t Wr = make_rsrc(W, w_row * static_cast<uint32_t>(N));
  const rsrc_t Ar = make_rsrc(A, a_row * static_cast<uint32_t>(M));
  StageOffsets<QT, MT> so;
  stage_offsets<QT, MT>(so, n0, N, M, w_row, a_row, lane, tid);

  f32x4 acc[MT];   // result, rows 4*kq + i, column l16
  f32x4 accm[MT];  // Q4_K: sum of (dmin*m) * s, subtracted at the end
#pragma unroll
  for (int a = 0; a < MT; ++a) acc[a] = accm[a] = f32x4{0.f, 0.f, 0.f, 0.f};

  // compute one super-block from the stage buffer at `as`
  auto compute = [&](const uint8_t *as) {
    const uint8_t *ws = as + S::kABytes + wave * S::kWBytes;
    // weight scales of this lane's column (row l16 of the n-tile)
    const uint8_t *row = ws + l16 * F::kPitch;
    float dsup = 0.0f;
    uint32_t scw[4] = {0, 0, 0, 0};
    if constexpr (QT == kTypeQ4_K) {
      const u32x4 hdr = *reinterpret_cast<const u32x4 *>(row);
      dsup = h2f(hdr.x & 0xFFFFu);
      scw[0] = hdr.y & 0x3F3F3F3Fu;                                          // sc 0-3
      scw[1] = (hdr.w & 0x0F0F0F0Fu) | ((hdr.y >> 2) & 0x30303030u);         // sc 4-7
      scw[2] = hdr.z & 0x3F3F3F3Fu;                                          // m 0-3
      scw[3] = ((hdr.w >> 4) & 0x0F0F0F0Fu) | ((hdr.z >> 2) & 0x30303030u);  // m 4-7
      // min term: sum over the 8 blocks of (dmin*m)[n] * s[m], as two fp32
      // MFMA 16x16x4 steps (K = blocks 4j..4j+3; this lane supplies k = kq)
      const float dmin = h2f(hdr.x >> 16);
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const float fm = dmin * static_cast<float>((scw[2 + j] >> (8 * kq)) & 0xFFu);
#pragma unroll
        for (int s = 0; s < MT; ++s) {
          const uint32_t ds = *reinterpret_cast<const uint32_t *>(
              as + (16 * s + l16) * kApitch + (4 * j + kq) * kQ8_1Bytes);
          accm[s] = __builtin_amdgcn_mfma_f32_16x16x4f32(h2f(ds >> 16), fm, accm[s], 0, 0, 0);
        }
      }
    } else if constexpr (QT == kTypeQ6_K) {
      dsup = h2f(*reinterpret_cast<const uint16_t *>(row + 208));
      const u32x4 sc = *reinterpret_cast<const u32x4 *>(row + 192);
      scw[0] = sc.x; scw[1] = sc.y; scw[2] = sc.z; scw[3] = sc.w;
    }
    // 64-bit views of the scale bytes: byte selects become shifts, not
    // indexed loads (keeps them in registers)
    const uint64_t sc8lo = static_cast<uint64_t>(scw[0]) | (static_cast<uint64_t>(scw[1]) << 32);
    const uint64_t sc8hi = static_cast<uint64_t>(scw[2]) | (static_cast<uint64_t>(scw[3]) << 32);

    f32x4 P[MT];  // super-block partial in units of the super-block d
#pragma unroll
    for (int a = 0; a < MT; ++a) P[a] = f32x4{0.f, 0.f, 0.f, 0.f};

#pragma unroll 2
    for (int b = 0; b < 8; ++b) {
      int64_t av[MT];
      float fa[MT][4];  // activation d of result rows 4*kq + i
#pragma unroll
      for (int s = 0; s < MT; ++s) {
        av[s] = ldg<int64_t>(as + (16 * s + l16) * kApitch + b * kQ8_1Bytes + 4 + 8 * kq);
#pragma unroll
        for (int i = 0; i < 4; ++i)
          fa[s][i] = h2f(*reinterpret_cast<const uint16_t *>(
              as + (16 * s + 4 * kq + i) * kApitch + b * kQ8_1Bytes));
      }
      if constexpr (QT == kTypeQ4_K) {
        const u32x2 q = *reinterpret_cast<const u32x2 *>(row + 16 + 32 * (b >> 1) + 8 * kq);
        const int sh = (b & 1) * 4;
        const int64_t bw = pack64((q.x >> sh) & 0x0F0F0F0Fu, (q.y >> sh) & 0x0F0F0F0Fu);
        const int sc = static_cast<int>((sc8lo >> (8 * b)) & 0xFFu);
#pragma unroll
        for (int s = 0; s < MT; ++s) {
          const i32x4 c = mfma16x16x32(av[s], bw);
#pragma unroll
          for (int i = 0; i < 4; ++i) P[s][i] += static_cast<float>(__mul24(c[i], sc)) * fa[s][i];
        }
      } else if constexpr (QT == kTypeQ6_K) {
        const int g = b >> 2, sub = b & 3;
        const u32x2 ql = *reinterpret_cast<const u32x2 *>(row + 64 * g + 32 * (sub & 1) + 8 * kq);
        const u32x2 qh = *reinterpret_cast<const u32x2 *>(row + 128 + 32 * g + 8 * kq);
        const int lsh = (sub >= 2) ? 4 : 0, hsh = 2 * sub;
        const uint32_t v0 = q6_minus32(((ql.x >> lsh) & 0x0F0F0F0Fu) | (((qh.x >> hsh) & 0x03030303u) << 4));
        const uint32_t v1 = q6_minus32(((ql.y >> lsh) & 0x0F0F0F0Fu) | (((qh.y >> hsh) & 0x03030303u) << 4));
        // values 0-15 come from lanes kq 0, 1; 16-31 from kq 2, 3: two MFMAs
        // so each half gets its own int8 scale (scales[g*8 + 2*sub + 0/1])
        const bool first = kq < 2;
        const int64_t bw0 = first ? pack64(v0, v1) : 0, bw1 = first ? 0 : pack64(v0, v1);
        const uint32_t two = static_cast<uint32_t>((g == 0 ? sc8lo : sc8hi) >> (16 * sub));
        const int sc0 = static_cast<int8_t>(two & 0xFFu);
        const int sc1 = static_cast<int8_t>((two >> 8) & 0xFFu);
#pragma unroll
        for (int s = 0; s < MT; ++s) {
          const i32x4 c0 = mfma16x16x32(av[s], bw0);
          const i32x4 c1 = mfma16x16x32(av[s], bw1);
#pragma unroll
          for (int i = 0; i < 4; ++i)
            P[s][i] += static_cast<float>(__mul24(c0[i], sc0) + __mul24(c1[i], sc1)) * fa[s][i];
        }
      } else {
        const uint8_t *blk = row + 34 * b;
        const float dw = h2f(ldg<uint16_t>(blk));
        const int64_t bw = ldg<int64_t>(blk + 2 + 8 * kq);
#pragma unroll
        for (int s = 0; s < MT; ++s) {
          const i32x4 c = mfma16x16x32(av[s], bw);
#pragma unroll
          for (int i = 0; i < 4; ++i) P[s][i] += static_cast<float>(c[i]) * (dw * fa[s][i]);
        }
      }
    }
#pragma unroll
    for (int a = 0; a < MT; ++a) {
      if constexpr (QT == kTypeQ8_0) acc[a] += P[a];
      else acc[a] += dsup * P[a];
    }
    };

  // r1 / r2: the two super-blocks in flight.  Before step s, super-block s
  // is committed to buf[s & 1] (visible after the step's barrier), s + 1 is
  // in one register set and s + 2 in the other, alternating.
  StageRegs<QT, MT> r1, r2;
  if (sb0 < sb1) {
    load_stage<QT, MT>(r1, so, Wr, Ar, sb0, lane, tid);
    if (sb0 + 1 < sb1) load_stage<QT, MT>(r2, so, Wr, Ar, sb0 + 1, lane, tid);
    store_stage<QT, MT>(buf[0], buf[0] + S::kABytes + wave * S::kWBytes, r1, lane, tid);
    if (sb0 + 2 < sb1) load_stage<QT, MT>(r1, so, Wr, Ar, sb0 + 2, lane, tid);
  }
  auto step = [&](int sb, int k, StageRegs<QT, MT> &rc) {
    __syncthreads();  // buf[k] complete; buf[k ^ 1] no longer read
    if (sb + 1 < sb1) {
      uint8_t *b = buf[k ^ 1];
      store_stage<QT, MT>(b, b + S::kABytes + wave * S::kWBytes, rc, lane, tid);
      if (sb + 3 < sb1) load_stage<QT, MT>(rc, so, Wr, Ar, sb + 3, lane, tid);
    }
    compute(buf[k]);
  };
  for (int sb = sb0; sb < sb1; sb += 2) {
    step(sb, 0, r2);
    if (sb + 1 < sb1) step(sb + 1, 1, r1);
  }
#pragma unroll
  for (int a = 0; a < MT; ++a) acc[a] -= accm[a];

  // ---- epilogue: lane holds column n and rows 4*kq + i of each m-tile
  const int n = n0 + l16;
  if (n >= N) return;
#pragma unroll
  for (int a = 0; a < MT; ++a)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int m = 16 * a + 4 * kq + i;
      if (m >= M) continue;
      const int64_t o = static_cast<int64_t>(m) * N + n;
      float y = acc[a][i];
      if constexpr (ATOMIC) {
        // Y was zeroed (store/bias) or holds the accumulate base
        if (mode == 2 && blockIdx.y == 0) y += static_cast<const float *>(bias)[n];
        atomicAdd(static_cast<float *>(Y) + o, y);
      } else if constexpr (F16OUT) {
        uint16_t *Yh = static_cast<uint16_t *>(Y);
        if (mode == 1) y += h2f(Yh[o]);
        else if (mode == 2) y += h2f(static_cast<const uint16_t *>(bias)[n]);
        Yh[o] = static_cast<uint16_t>(f2h_bits(y));
      } else {
        float *Yf = static_cast<float *>(Y);
        if (mode == 1) y += Yf[o];
        else if (mode == 2) y += static_cast<const float *>(bias)[n];
        Yf[o] = y;
      }
    }
}

namespace {

// Super-block splits: enough workgroups for ~16 waves per CU, at least two
// super-blocks per split.  IFX_SKINNY_SPLIT overrides (tuning; read once).
int choose_splits(int row_groups, int nsb) {
  static const int env = [] {
    const char *e = ifx::tuning_env("IFX_SKINNY_SPLIT");
    return e ? atoi(e) : 0;
  }();
  int ks = env > 0 ? env : (1024 + row_groups - 1) / row_groups;
  ks = max(1, min(ks, nsb / 2 > 0 ? nsb / 2 : 1));
  return ks;
}

template <int QT, int MT>
hipError_t launch_mt(SkArgs args, bool f16, hipStream_t s) {
  constexpr int shm = 2 * Stage<QT, MT>::kBytes;
  int groups = 0;
  for (int i = 0; i < args.nseg; ++i) {
    args.seg[i].blk_begin = groups;
    groups += (args.seg[i].N + 16 * kWaves - 1) / (16 * kWaves);
  }
  const int nsb = args.K >> 8;
  int ks = f16 ? 1 : choose_splits(groups, nsb);
  args.sb_per = (nsb + ks - 1) / ks;
  ks = (nsb + args.sb_per - 1) / args.sb_per;
  const dim3 grid(groups, ks);
  if (f16) {
    IFX_LAUNCH(k_mmq_skinny, (QT, MT, true, false), grid, dim3(64 * kWaves), shm, s, args);
  } else if (ks == 1) {
    IFX_LAUNCH(k_mmq_skinny, (QT, MT, false, false), grid, dim3(64 * kWaves), shm, s, args);
  } else {
    if (args.mode != 1) {  // store / bias: the splits add into zeroed outputs
      FillArgs f{};
      for (int i = 0; i < args.nseg; ++i) {
        f.y[i] = static_cast<float *>(args.seg[i].Y);
        f.n[i] = static_cast<int64_t>(args.M) * args.seg[i].N;
      }
      if (launch_fill_zero(f, args.nseg, s) != hipSuccess) return last_error();
    }
    IFX_LAUNCH(k_mmq_skinny, (QT, MT, false, true), grid, dim3(64 * kWaves), shm, s, args);
  }
  return last_error();
}

}  // namespace

// Requires K % 256 == 0 and 1 <= M <= 32 (checked by the caller).  count
// projections (1..3) of one quant type share A; bias only with count == 1.
hipError_t launch_mmq_skinny(int qtype, int count, const void *const *W, void *const *Y,
                             const int *N, const void *bias, const void *A, bool f16, int M,
                             int K, int mode, hipStream_t stream) {
  if (M > 32 || count < 1 || count > 3) return hipErrorInvalidValue;
  SkArgs args{};
  for (int i = 0; i < count; ++i)
    args.seg[i] = SkSeg{static_cast<const uint8_t *>(W[i]), Y[i], i == 0 ? bias : nullptr, N[i], 0};
  args.nseg = count;
  args.A = static_cast<const uint8_t *>(A);
  args.M = M;
  args.K = K;
  args.mode = mode;
  const bool two = M > 16;  // two m-tiles of 16
  switch (qtype) {
  case kTypeQ4_K: return two ? launch_mt<kTypeQ4_K, 2>(args, f16, stream) : launch_mt<kTypeQ4_K, 1>(args, f16, stream);
  case kTypeQ6_K: return two ? launch_mt<kTypeQ6_K, 2>(args, f16, stream) : launch_mt<kTypeQ6_K, 1>(args, f16, stream);
  case kTypeQ8_0: return two ? launch_mt<kTypeQ8_0, 2>(args, f16, stream) : launch_mt<kTypeQ8_0, 1>(args, f16, stream);
  default: return hipErrorInvalidValue;
  }
}

}  // namespace ifx
