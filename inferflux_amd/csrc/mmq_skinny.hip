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
//  * A workgroup owns 16*NT weight rows and all (<= 32) batch rows; its KW
//    waves split the super-blocks (256 values of K) round-robin, so small-N
//    projections still fill the chip, and add their partial sums in LDS in
//    a fixed order (deterministic results).
//  * Per super-block each wave copies its W rows and A rows into its own
//    LDS region with 16-byte loads whose lanes cover contiguous memory (the
//    raw bytes: 144 B Q4_K, 210 B Q6_K, 8 x 34 B Q8_0 per row; 8 x 36 B
//    Q8_1), then reads the MFMA operands from LDS.
//  * Scaling: Q4_K and Q6_K sub-block scales are integers, so each block's
//    int32 result is multiplied by its scale in the integer pipe and the
//    fp32 sum is taken in units of the super-block d (one multiply by d per
//    super-block).  The Q4_K min term sum_b (dmin*m_b) * s_b is a small
//    fp32 GEMM done on the matrix cores (v_mfma_f32_16x16x4f32).
#include "ifx_common.h"

#include <stdlib.h>

namespace ifx {

namespace {

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
  static constexpr int kBytes = 144, kPitch = 144, kChunks = 9;
};
template <>
struct WFmt<kTypeQ6_K> {  // 210 raw bytes; the 14th chunk carries only d
  static constexpr int kBytes = 210, kPitch = 224, kChunks = 14;
};
template <>
struct WFmt<kTypeQ8_0> {  // 8 blocks x 34 bytes
  static constexpr int kBytes = 272, kPitch = 272, kChunks = 17;
};

constexpr int kApitch = 288;  // 8 Q8_1 blocks x 36 bytes
constexpr int kAChunks = 18;

template <int QT, int MT, int NT>
struct Stage {
  static constexpr int kWBytes = 16 * NT * WFmt<QT>::kPitch;
  static constexpr int kABytes = 16 * MT * kApitch;
  static constexpr int kBytes = kWBytes + kABytes;
  static constexpr int kWChunks = 16 * NT * WFmt<QT>::kChunks;
  static constexpr int kAChunksAll = 16 * MT * kAChunks;
  static constexpr int kWPerLane = (kWChunks + 63) / 64;
  static constexpr int kAPerLane = (kAChunksAll + 63) / 64;
};

// This lane's 16-byte chunks of one super-block's W rows and A rows.
template <int QT, int MT, int NT>
struct StageRegs {
  u32x4 w[Stage<QT, MT, NT>::kWPerLane];
  u32x4 a[Stage<QT, MT, NT>::kAPerLane];
};

// Per-lane byte offsets of this lane's 16-byte chunks within super-block 0
// (loop invariant; super-block sb adds sb * bytes-per-super-block).  Rows
// past N repeat row N-1; chunks of rows past M get offset -1 (zero fill).
template <int QT, int MT, int NT>
struct StageOffsets {
  uint32_t w[Stage<QT, MT, NT>::kWPerLane];
  int32_t a[Stage<QT, MT, NT>::kAPerLane];
};

template <int QT, int MT, int NT>
__device__ __forceinline__ void stage_offsets(StageOffsets<QT, MT, NT> &so, int n0, int N, int M,
                                              int nsb, int nblk, int lane) {
  using S = Stage<QT, MT, NT>;
  using F = WFmt<QT>;
  const uint32_t wrow = (QT == kTypeQ8_0) ? static_cast<uint32_t>(nblk) * kQ8_0Bytes
                                          : static_cast<uint32_t>(nsb) * F::kBytes;
#pragma unroll
  for (int i = 0; i < S::kWPerLane; ++i) {
    const int c = min(lane + 64 * i, S::kWChunks - 1);
    const int r = c / F::kChunks, part = c - r * F::kChunks;
    so.w[i] = static_cast<uint32_t>(min(n0 + r, N - 1)) * wrow + part * 16;
  }
#pragma unroll
  for (int i = 0; i < S::kAPerLane; ++i) {
    const int c = min(lane + 64 * i, S::kAChunksAll - 1);
    const int r = c / kAChunks, part = c - r * kAChunks;
    so.a[i] = (r < M) ? r * nblk * kQ8_1Bytes + part * 16 : -1;
  }
}

// Global -> registers: this lane's chunks of super-block sb, as buffer
// loads (per-lane 32-bit offset + wave-uniform super-block offset).
template <int QT, int MT, int NT>
__device__ __forceinline__ void load_stage(StageRegs<QT, MT, NT> &rg,
                                           const StageOffsets<QT, MT, NT> &so, rsrc_t Wr,
                                           rsrc_t Ar, int sb, int lane) {
  using S = Stage<QT, MT, NT>;
  using F = WFmt<QT>;
  const uint32_t wsb = sb * (QT == kTypeQ8_0 ? 8 * kQ8_0Bytes : F::kBytes);
  const uint32_t asb = sb * (8 * kQ8_1Bytes);
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
  for (int i = 0; i < S::kAPerLane; ++i) {
    const int c = lane + 64 * i;
    rg.a[i] = u32x4{0, 0, 0, 0};
    if ((S::kAChunksAll % 64 == 0 || i + 1 < S::kAPerLane || c < S::kAChunksAll) && so.a[i] >= 0)
      rg.a[i] = bload<u32x4>(Ar, static_cast<uint32_t>(so.a[i]), asb);
  }
}

template <int QT, int MT, int NT>
__device__ __forceinline__ void store_stage(uint8_t *st, const StageRegs<QT, MT, NT> &rg,
                                            int lane) {
  using S = Stage<QT, MT, NT>;
  using F = WFmt<QT>;
#pragma unroll
  for (int i = 0; i < S::kWPerLane; ++i) {
    const int c = lane + 64 * i;
    if (c < S::kWChunks) {
      const int r = c / F::kChunks, part = c - r * F::kChunks;
      *reinterpret_cast<u32x4 *>(st + r * F::kPitch + part * 16) = rg.w[i];
    }
  }
  uint8_t *as = st + S::kWBytes;
#pragma unroll
  for (int i = 0; i < S::kAPerLane; ++i) {
    const int c = lane + 64 * i;
    if (c < S::kAChunksAll) *reinterpret_cast<u32x4 *>(as + c * 16) = rg.a[i];
  }
}

}  // namespace

template <int QT, int MT, int NT, int KW, bool F16OUT>
__global__ __launch_bounds__(64 * KW, 4) void k_mmq_skinny(const uint8_t *__restrict__ W,
                                                        const uint8_t *__restrict__ A,
                                                        void *__restrict__ Y,
                                                        const void *__restrict__ bias, int M,
                                                        int N, int K, int mode) {
  using S = Stage<QT, MT, NT>;
  using F = WFmt<QT>;
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const int lane = threadIdx.x & 63;
  // wave-uniform values kept in scalar registers
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int l16 = lane & 15, kq = lane >> 4;
  const int n0 = blockIdx.x * 16 * NT;
  const int m0 = 0;
  const int nblk = K >> 5;  // Q8_1 blocks per activation row
  const int nsb = K >> 8;   // super-blocks of 256 values
  uint8_t *st = smem + wave * S::kBytes;       // this wave's W rows
  const uint8_t *as = st + S::kWBytes;         // this wave's A rows

  f32x4 acc[MT][NT];   // result, rows 4*kq + i, column l16
  f32x4 accm[MT][NT];  // Q4_K: sum of (dmin*m) * s, subtracted at the end
#pragma unroll
  for (int a = 0; a < MT; ++a)
#pragma unroll
    for (int b = 0; b < NT; ++b) acc[a][b] = accm[a][b] = f32x4{0.f, 0.f, 0.f, 0.f};

  StageOffsets<QT, MT, NT> so;
  stage_offsets<QT, MT, NT>(so, n0, N, M, nsb, nblk, lane);
  const uint32_t w_bytes = static_cast<uint32_t>(N) *
      (QT == kTypeQ8_0 ? static_cast<uint32_t>(nblk) * kQ8_0Bytes : static_cast<uint32_t>(nsb) * F::kBytes);
  const rsrc_t Wr = make_rsrc(W, w_bytes);
  const rsrc_t Ar = make_rsrc(A, static_cast<uint32_t>(M) * nblk * kQ8_1Bytes);
  // every wave runs the same number of iterations (the barriers need it);
  // the other waves on the CU cover each wave's load latency
  const int iters = (nsb + KW - 1) / KW;
  for (int it = 0; it < iters; ++it) {
    const int sb = it * KW + wave;
    {
      StageRegs<QT, MT, NT> rg;
      if (sb < nsb) load_stage<QT, MT, NT>(rg, so, Wr, Ar, sb, lane);
      __syncthreads();  // previous iteration's LDS reads are done
      if (sb < nsb) store_stage<QT, MT, NT>(st, rg, lane);
      __syncthreads();
    }
    if (sb >= nsb) continue;

    // weight scales of this lane's column (row l16 of each n-tile)
    float dsup[NT];
    uint32_t scw[NT][4];
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const uint8_t *row = st + (16 * t + l16) * F::kPitch;
      if constexpr (QT == kTypeQ4_K) {
        const u32x4 hdr = *reinterpret_cast<const u32x4 *>(row);
        dsup[t] = h2f(hdr.x & 0xFFFFu);
        scw[t][0] = hdr.y & 0x3F3F3F3Fu;                                            // sc 0-3
        scw[t][1] = (hdr.w & 0x0F0F0F0Fu) | ((hdr.y >> 2) & 0x30303030u);           // sc 4-7
        scw[t][2] = hdr.z & 0x3F3F3F3Fu;                                            // m 0-3
        scw[t][3] = ((hdr.w >> 4) & 0x0F0F0F0Fu) | ((hdr.z >> 2) & 0x30303030u);    // m 4-7
        // min term: sum over the 8 blocks of (dmin*m)[n] * s[m], as two fp32
        // MFMA 16x16x4 steps (K = blocks 4j..4j+3; this lane supplies k = kq)
        const float dmin = h2f(hdr.x >> 16);
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const float fm = dmin * static_cast<float>((scw[t][2 + j] >> (8 * kq)) & 0xFFu);
#pragma unroll
          for (int s = 0; s < MT; ++s) {
            const uint32_t ds = *reinterpret_cast<const uint32_t *>(
                as + (16 * s + l16) * kApitch + (4 * j + kq) * kQ8_1Bytes);
            accm[s][t] = __builtin_amdgcn_mfma_f32_16x16x4f32(h2f(ds >> 16), fm, accm[s][t], 0, 0, 0);
          }
        }
      } else if constexpr (QT == kTypeQ6_K) {
        dsup[t] = h2f(*reinterpret_cast<const uint16_t *>(row + 208));
        const u32x4 sc = *reinterpret_cast<const u32x4 *>(row + 192);
        scw[t][0] = sc.x; scw[t][1] = sc.y; scw[t][2] = sc.z; scw[t][3] = sc.w;
      }
    }

    f32x4 P[MT][NT];  // super-block partial in units of the super-block d
#pragma unroll
    for (int a = 0; a < MT; ++a)
#pragma unroll
      for (int b = 0; b < NT; ++b) P[a][b] = f32x4{0.f, 0.f, 0.f, 0.f};

    // two blocks per step: enough independent MFMAs to hide their latency
    // without hoisting all eight blocks' operands into registers
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
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        const uint8_t *row = st + (16 * t + l16) * F::kPitch;
        if constexpr (QT == kTypeQ4_K) {
          const u32x2 q = *reinterpret_cast<const u32x2 *>(row + 16 + 32 * (b >> 1) + 8 * kq);
          const int sh = (b & 1) * 4;
          const int64_t bw = pack64((q.x >> sh) & 0x0F0F0F0Fu, (q.y >> sh) & 0x0F0F0F0Fu);
          const int sc = static_cast<int>((scw[t][b >> 2] >> (8 * (b & 3))) & 0xFFu);
#pragma unroll
          for (int s = 0; s < MT; ++s) {
            const i32x4 c = mfma16x16x32(av[s], bw);
#pragma unroll
            for (int i = 0; i < 4; ++i) P[s][t][i] += static_cast<float>(c[i] * sc) * fa[s][i];
          }
        } else if constexpr (QT == kTypeQ6_K) {
          const int g = b >> 2, sub = b & 3;
          const u32x2 ql = *reinterpret_cast<const u32x2 *>(row + 64 * g + 32 * (sub & 1) + 8 * kq);
          const u32x2 qh = *reinterpret_cast<const u32x2 *>(row + 128 + 32 * g + 8 * kq);
          const int lsh = (sub >= 2) ? 4 : 0, hsh = 2 * sub;
          const uint32_t v0 = q6_minus32(((ql.x >> lsh) & 0x0F0F0F0Fu) | (((qh.x >> hsh) & 0x03030303u) << 4));
          const uint32_t v1 = q6_minus32(((ql.y >> lsh) & 0x0F0F0F0Fu) | (((qh.y >> hsh) & 0x03030303u) << 4));
          // values 0-15 come from lanes kq 0, 1; 16-31 from kq 2, 3: two
          // MFMAs so each half gets its own int8 scale
          const bool first = kq < 2;
          const int64_t bw0 = first ? pack64(v0, v1) : 0, bw1 = first ? 0 : pack64(v0, v1);
          const int si = g * 8 + 2 * sub;  // even: both halves' scales in one dword
          const uint32_t hw = scw[t][si >> 2];
          const int sc0 = static_cast<int8_t>((hw >> (8 * (si & 3))) & 0xFFu);
          const int sc1 = static_cast<int8_t>((hw >> (8 * ((si & 3) + 1))) & 0xFFu);
#pragma unroll
          for (int s = 0; s < MT; ++s) {
            const i32x4 c0 = mfma16x16x32(av[s], bw0);
            const i32x4 c1 = mfma16x16x32(av[s], bw1);
#pragma unroll
            for (int i = 0; i < 4; ++i)
              P[s][t][i] += static_cast<float>(c0[i] * sc0 + c1[i] * sc1) * fa[s][i];
          }
        } else {
          const uint8_t *blk = row + 34 * b;
          const float dw = h2f(ldg<uint16_t>(blk));
          const int64_t bw = ldg<int64_t>(blk + 2 + 8 * kq);
#pragma unroll
          for (int s = 0; s < MT; ++s) {
            const i32x4 c = mfma16x16x32(av[s], bw);
#pragma unroll
            for (int i = 0; i < 4; ++i) P[s][t][i] += static_cast<float>(c[i]) * (dw * fa[s][i]);
          }
        }
      }
    }
#pragma unroll
    for (int a = 0; a < MT; ++a)
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        if constexpr (QT == kTypeQ8_0) acc[a][t] += P[a][t];
        else acc[a][t] += dsup[t] * P[a][t];
      }
  }
#pragma unroll
  for (int a = 0; a < MT; ++a)
#pragma unroll
    for (int t = 0; t < NT; ++t) acc[a][t] -= accm[a][t];

  // ---- combine the KW waves' partial sums in a fixed order (LDS reused)
  if constexpr (KW > 1) {
    constexpr int NACC = MT * NT * 4;
    float *red = reinterpret_cast<float *>(smem);
    __syncthreads();
    if (wave > 0) {
      float *dst = red + ((wave - 1) * NACC) * 64 + lane;
#pragma unroll
      for (int a = 0; a < MT; ++a)
#pragma unroll
        for (int b = 0; b < NT; ++b)
#pragma unroll
          for (int i = 0; i < 4; ++i) dst[((a * NT + b) * 4 + i) * 64] = acc[a][b][i];
    }
    __syncthreads();
    if (wave > 0) return;
#pragma unroll
    for (int w = 0; w < KW - 1; ++w) {
      const float *src = red + (w * NACC) * 64 + lane;
#pragma unroll
      for (int a = 0; a < MT; ++a)
#pragma unroll
        for (int b = 0; b < NT; ++b)
#pragma unroll
          for (int i = 0; i < 4; ++i) acc[a][b][i] += src[((a * NT + b) * 4 + i) * 64];
    }
  }

  // ---- epilogue: lane holds column n and rows 4*kq + i of each tile
#pragma unroll
  for (int b = 0; b < NT; ++b) {
    const int n = n0 + 16 * b + l16;
    if (n >= N) continue;
#pragma unroll
    for (int a = 0; a < MT; ++a)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int m = m0 + 16 * a + 4 * kq + i;
        if (m >= M) continue;
        const int64_t o = static_cast<int64_t>(m) * N + n;
        float y = acc[a][b][i];
        if constexpr (F16OUT) {
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
}

namespace {

constexpr int kMaxLds = 160 * 1024;

template <int QT, int MT, int NT, int KW>
hipError_t launch_k(const uint8_t *W, const uint8_t *A, void *Y, const void *bias, bool f16, int M,
                    int N, int K, int mode, hipStream_t s) {
  using St = Stage<QT, MT, NT>;
  constexpr int stage = KW * St::kBytes;
  constexpr int red = (KW > 1) ? (KW - 1) * MT * NT * 4 * 64 * 4 : 0;
  constexpr int shm = stage > red ? stage : red;
  static_assert(shm <= kMaxLds, "LDS budget");
  auto kern = f16 ? k_mmq_skinny<QT, MT, NT, KW, true> : k_mmq_skinny<QT, MT, NT, KW, false>;
  static bool attr_set[2] = {false, false};
  if (shm > 64 * 1024 && !attr_set[f16]) {
    const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void *>(kern),
                                             hipFuncAttributeMaxDynamicSharedMemorySize, shm);
    if (e != hipSuccess) return e;
    attr_set[f16] = true;
  }
  const dim3 grid((N + 16 * NT - 1) / (16 * NT));
  hipLaunchKernelGGL(kern, grid, dim3(64 * KW), shm, s, W, A, Y, bias, M, N, K, mode);
  return hipGetLastError();
}

template <int QT, int MT, int NT>
hipError_t launch_kw(const uint8_t *W, const uint8_t *A, void *Y, const void *bias, bool f16,
                     int M, int N, int K, int mode, hipStream_t s) {
  // enough waves to cover the chip (~16 per CU) without splitting K finer
  // than one super-block per wave, within the LDS budget
  using St = Stage<QT, MT, NT>;
  const int tiles = (N + 16 * NT - 1) / (16 * NT);
  const int nsb = K >> 8;
  int kw = 1;
  while (kw < 16 && kw * 2 <= nsb && tiles * kw < 4096 && (2 * kw) * St::kBytes <= kMaxLds)
    kw *= 2;
  static const int kw_env = [] {
    const char *e = getenv("IFX_SKINNY_KW");
    return e ? atoi(e) : 0;
  }();
  if (kw_env > 0 && kw_env <= nsb && kw_env * St::kBytes <= kMaxLds) kw = kw_env;
  switch (kw) {
  case 1: return launch_k<QT, MT, NT, 1>(W, A, Y, bias, f16, M, N, K, mode, s);
  case 2: return launch_k<QT, MT, NT, 2>(W, A, Y, bias, f16, M, N, K, mode, s);
  case 4: return launch_k<QT, MT, NT, 4>(W, A, Y, bias, f16, M, N, K, mode, s);
  case 8: return launch_k<QT, MT, NT, 8>(W, A, Y, bias, f16, M, N, K, mode, s);
  default:
    if constexpr (16 * St::kBytes <= kMaxLds)
      return launch_k<QT, MT, NT, 16>(W, A, Y, bias, f16, M, N, K, mode, s);
    else
      return launch_k<QT, MT, NT, 8>(W, A, Y, bias, f16, M, N, K, mode, s);
  }
}

}  // namespace

// Requires K % 256 == 0 and 1 <= M <= 32 (checked by the caller).
hipError_t launch_mmq_skinny(int qtype, const void *W, const void *A, void *Y, const void *bias,
                             bool f16, int M, int N, int K, int mode, hipStream_t stream) {
  const uint8_t *w = static_cast<const uint8_t *>(W);
  const uint8_t *a = static_cast<const uint8_t *>(A);
  if (M > 32) return hipErrorInvalidValue;
  const bool two = M > 16;  // two m-tiles of 16
  switch (qtype) {
  case kTypeQ4_K:
    return two ? launch_kw<kTypeQ4_K, 2, 2>(w, a, Y, bias, f16, M, N, K, mode, stream)
               : launch_kw<kTypeQ4_K, 1, 2>(w, a, Y, bias, f16, M, N, K, mode, stream);
  case kTypeQ6_K:
    return two ? launch_kw<kTypeQ6_K, 2, 1>(w, a, Y, bias, f16, M, N, K, mode, stream)
               : launch_kw<kTypeQ6_K, 1, 1>(w, a, Y, bias, f16, M, N, K, mode, stream);
  case kTypeQ8_0:
    return two ? launch_kw<kTypeQ8_0, 2, 1>(w, a, Y, bias, f16, M, N, K, mode, stream)
               : launch_kw<kTypeQ8_0, 1, 1>(w, a, Y, bias, f16, M, N, K, mode, stream);
  default: return hipErrorInvalidValue;
  }
}

}  // namespace ifx
