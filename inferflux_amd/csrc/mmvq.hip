// mmvq.hip -- decode-batch quantized GEMV on the gfx950 matrix cores, for
// 1 <= M <= 32: y[m][n] = sum_k W[n][k] * a[m][k], W raw GGUF Q4_K / Q6_K /
// Q8_0 blocks, a Q8_1 blocks of 32.
//
// Replaces the reference's MMVQ and MMQ decode kernels
// (runtime/backends/cuda/native/kernels/mmvq.cuh:49-1019 for M <= 8,
// kernels/mmq.cuh:41-835 for 9 <= M <= 64) and their grouped pair/triple
// launches (mmvq.cuh:1197-1448).  The arithmetic is the reference's: an
// exact integer dot per 32-value block (two 16-value halves for Q6_K), then
// fp32 scaling by the weight and activation block scales; the Q4_K min term
// uses the Q8_1 s = d * sum(q) field (mmvq.cuh:115-125, 467-471, 886-889).
//
// Mapping.  One v_mfma_i32_16x16x32_i8 multiplies a 16 (batch rows m) x 32
// tile of activation codes by a 32 x 16 (weight rows n) tile of weight
// codes.  Lane l supplies batch row l % 16 and weight row l % 16 for the
// 8-value K chunk q = l / 16, and receives weight row n = l % 16 and batch
// rows 4q + i (i < 4) of the block's int32 dot products.  So
//  * the K reduction inside a block happens in the matrix core (no
//    cross-lane shuffles);
//  * a lane's weight scales are those of its own row n, which it loads
//    itself (one 16-byte header load per super-block);
//  * batch rows past M are zero operands, so one code path serves M = 1..16
//    (MT = 1) and 17..32 (MT = 2 tiles of 16); the matrix cores are idle
//    otherwise, the padding costs no time that the weight stream does not
//    already take.
// The activation d of batch rows 4q + i is exchanged through 512 bytes of
// LDS per tile (each lane loads two blocks' d of its own batch row).  The
// Q4_K min term sum_b (dmin*m[n][b]) * s[m][b] is two fp32 16x16x4 MFMAs per
// super-block.
//
// Work split.  A workgroup owns 16 weight rows of one projection and has KW
// waves; wave w walks super-blocks w, w + KW, ... (256 values of K; for Q8_0
// eight blocks of 32), loading the next one before computing the current.
// The KW partial tiles are summed through LDS and stored once -- no atomics,
// every output written by exactly one lane, deterministic.  KW grows as N
// shrinks so that the chip has several thousand waves in flight.
// Workgroups walk the rows of up to three projections that read the same
// activations (grouped launches), as the GEMV kernel does.
#include "ifx_common.h"

#include <stdlib.h>

namespace ifx {

enum MmvqOutMode { kMvStore = 0, kMvAccum = 1, kMvBias = 2 };

struct MmvqSeg {
  const uint8_t *W;
  void *Y;
  const void *bias;
  int N;
  int blk_begin;
};

struct MmvqArgs {
  MmvqSeg seg[3];
  int nseg;
  const uint8_t *A;
  int M, K, mode;
};

namespace {

__device__ __forceinline__ i32x4 mfma_i8(int64_t a, int64_t b) {
  const i32x4 z = {0, 0, 0, 0};
  return __builtin_amdgcn_mfma_i32_16x16x32_i8(a, b, z, 0, 0, 0);
}

__device__ __forceinline__ int64_t pack64(uint32_t lo, uint32_t hi) {
  return static_cast<int64_t>(static_cast<uint64_t>(lo) | (static_cast<uint64_t>(hi) << 32));
}

// Q6_K code bytes v in [0, 63] -> int8 (v - 32), four per dword, no carries:
// flip bit 5, then copy the new bit 5 into bits 6 and 7.
__device__ __forceinline__ uint32_t q6_minus32(uint32_t v) {
  const uint32_t x = v ^ 0x20202020u;
  const uint32_t t = x & 0x20202020u;
  return x | (t << 1) | (t << 2);
}

// Weight bytes of one super-block held by a lane (its own row n, K chunk q).
template <int QT>
struct WRegs;
template <>
struct WRegs<kTypeQ4_K> {
  u32x4 hdr;   // d, dmin, scales[12]
  u32x2 q[4];  // qs[32g + 8q .. +8], g = 0..3
};
template <>
struct WRegs<kTypeQ6_K> {
  u32x2 ql[4];  // ql[64g + 32h + 8q .. +8], index 2g + h
  u32x2 qh[2];  // qh[32g + 8q .. +8]
  u32x4 sc;     // scales[16]
  uint32_t d;   // fp16 bits
};
template <>
struct WRegs<kTypeQ8_0> {
  u32x2 q[8];    // block b codes [8q .. +8]
  uint32_t d[8]; // block b fp16 d
};

template <int MT>
struct ARegs {
  int64_t c[MT][8];   // batch row 16t + l16, block b, codes [8q .. +8]
  uint32_t ds[MT][2]; // batch row 16t + l16, blocks q and q + 4: d | s << 16
};

// Raw bytes of one super-block of a weight row, as staged in LDS.
template <int QT>
struct WFmt;
template <>
struct WFmt<kTypeQ4_K> {  // 144 bytes = 9 chunks of 16
  static constexpr int kSb = 144, kPitch = 144, kChunks = 9;
};
template <>
struct WFmt<kTypeQ6_K> {  // 210 bytes; the 14th chunk carries d (2 bytes)
  static constexpr int kSb = 210, kPitch = 224, kChunks = 14;
};
template <>
struct WFmt<kTypeQ8_0> {  // 8 blocks x 34 bytes
  static constexpr int kSb = 272, kPitch = 272, kChunks = 17;
};
constexpr int kAChunks = 18;  // 8 Q8_1 blocks of 36 bytes per batch row
constexpr int kAPitch = 304;  // + 16: rows start on distinct LDS banks

// Per-wave LDS: this super-block's 16 weight rows and batch rows.
template <int QT, int MT>
struct WaveLds {
  uint8_t w[16 * WFmt<QT>::kPitch];
  uint8_t a[MT * 16 * kAPitch];
  float dl[MT][8][16];  // activation d, [tile][block][batch row]
};

// One super-block's 16-byte chunks in flight in a lane's registers.
template <int QT, int MT>
struct Chunks {
  static constexpr int kW = (16 * WFmt<QT>::kChunks + 63) / 64;
  static constexpr int kA = (MT * 16 * kAChunks + 63) / 64;
  u32x4 w[kW];
  u32x4 a[kA];
};

// A 16-byte chunk at byte offset off of a tensor of `end` bytes.  A buffer
// load that crosses the end of its range returns zeros for all of it, so
// the (at most one per tensor) chunk that straddles the end is read in
// G-byte pieces; G divides every row length (2 for weights, 4 for Q8_1).
template <int G, bool W>
__device__ __forceinline__ u32x4 load16_clip(rsrc_t r, uint32_t off, uint32_t end) {
  if (off + 16 <= end) return W ? wload<u32x4>(r, off, 0) : bload<u32x4>(r, off, 0);
  uint32_t v[4] = {0, 0, 0, 0};
#pragma unroll
  for (int k = 0; k < 16 / G; ++k) {
    const uint32_t o = off + G * k;
    if (o < end) {
      const uint32_t x = (G == 2) ? bload<uint16_t>(r, o, 0) : bload<uint32_t>(r, o, 0);
      v[(G * k) >> 2] |= x << (8 * ((G * k) & 3));
    }
  }
  return u32x4{v[0], v[1], v[2], v[3]};
}

// Global -> registers: chunk c of the weight tile is row c / kChunks, part
// c % kChunks; consecutive lanes read consecutive 16 bytes of a row.
template <int QT, int MT>
__device__ __forceinline__ void fetch(Chunks<QT, MT> &ch, rsrc_t Wr, rsrc_t Ar, int n0, int N,
                                      int M, uint32_t w_row, uint32_t a_row, int sb, int lane) {
  using F = WFmt<QT>;
#pragma unroll
  for (int i = 0; i < Chunks<QT, MT>::kW; ++i) {
    const int c = lane + 64 * i;
    ch.w[i] = u32x4{0, 0, 0, 0};
    if (c < 16 * F::kChunks) {
      const int r = c / F::kChunks, part = c - r * F::kChunks;
      const uint32_t row = static_cast<uint32_t>(min(n0 + r, N - 1));
      ch.w[i] = load16_clip<2, true>(Wr, row * w_row + sb * F::kSb + 16 * part, w_row * static_cast<uint32_t>(N));
    }
  }
#pragma unroll
  for (int i = 0; i < Chunks<QT, MT>::kA; ++i) {
    const int c = lane + 64 * i;
    ch.a[i] = u32x4{0, 0, 0, 0};
    if (c < M * kAChunks) {
      const int r = c / kAChunks, part = c - r * kAChunks;
      ch.a[i] = load16_clip<4, false>(Ar, r * a_row + sb * (8 * kQ8_1Bytes) + 16 * part, a_row * static_cast<uint32_t>(M));
    }
  }
}

// Registers -> this wave's LDS slot.
template <int QT, int MT>
__device__ __forceinline__ void commit(WaveLds<QT, MT> &L, const Chunks<QT, MT> &ch, int M,
                                       int lane) {
  using F = WFmt<QT>;
#pragma unroll
  for (int i = 0; i < Chunks<QT, MT>::kW; ++i) {
    const int c = lane + 64 * i;
    if (c < 16 * F::kChunks) {
      const int r = c / F::kChunks, part = c - r * F::kChunks;
      *reinterpret_cast<u32x4 *>(L.w + r * F::kPitch + 16 * part) = ch.w[i];
    }
  }
#pragma unroll
  for (int i = 0; i < Chunks<QT, MT>::kA; ++i) {
    const int c = lane + 64 * i;
    if (c < M * kAChunks) {
      const int r = c / kAChunks, part = c - r * kAChunks;
      *reinterpret_cast<u32x4 *>(L.a + r * kAPitch + 16 * part) = ch.a[i];
    }
  }
}

__device__ __forceinline__ void wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// LDS -> MFMA operands of this lane (weight row l16, K chunk q).
template <int QT, int MT>
__device__ __forceinline__ void read_w(WRegs<QT> &w, const WaveLds<QT, MT> &L, int l16, int q,
                                       int sb, int nblk) {
  const uint8_t *row = L.w + l16 * WFmt<QT>::kPitch;
  if constexpr (QT == kTypeQ4_K) {
    w.hdr = *reinterpret_cast<const u32x4 *>(row);
#pragma unroll
    for (int g = 0; g < 4; ++g) w.q[g] = *reinterpret_cast<const u32x2 *>(row + 16 + 32 * g + 8 * q);
  } else if constexpr (QT == kTypeQ6_K) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
      w.ql[i] = *reinterpret_cast<const u32x2 *>(row + 64 * (i >> 1) + 32 * (i & 1) + 8 * q);
#pragma unroll
    for (int g = 0; g < 2; ++g) w.qh[g] = *reinterpret_cast<const u32x2 *>(row + 128 + 32 * g + 8 * q);
    w.sc = *reinterpret_cast<const u32x4 *>(row + 192);
    w.d = *reinterpret_cast<const uint16_t *>(row + 208);
  } else {
#pragma unroll
    for (int b = 0; b < 8; ++b) {
      const bool ok = sb * 8 + b < nblk;
      w.d[b] = ok ? ldg<uint16_t>(row + kQ8_0Bytes * b) : 0;
      w.q[b] = ok ? ldg<u32x2>(row + kQ8_0Bytes * b + 2 + 8 * q) : u32x2{0, 0};
    }
  }
}

template <int QT, int MT>
__device__ __forceinline__ void read_a(ARegs<MT> &a, const WaveLds<QT, MT> &L, const bool (&a_ok)[MT],
                                       int l16, int q, int sb, int nblk) {
#pragma unroll
  for (int t = 0; t < MT; ++t) {
    const uint8_t *row = L.a + (16 * t + l16) * kAPitch;
#pragma unroll
    for (int b = 0; b < 8; ++b)
      a.c[t][b] = (a_ok[t] && sb * 8 + b < nblk) ? ldg<int64_t>(row + kQ8_1Bytes * b + 4 + 8 * q) : 0;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int b = q + 4 * j;
      a.ds[t][j] = (a_ok[t] && sb * 8 + b < nblk) ? ldg<uint32_t>(row + kQ8_1Bytes * b) : 0;
    }
  }
}

}  // namespace

template <int QT, int MT, int KW>
constexpr int mmvq_lds_bytes() {
  constexpr int stage = KW * sizeof(WaveLds<QT, MT>);
  constexpr int red = (KW > 1 ? KW - 1 : 1) * MT * 64 * sizeof(f32x4);
  return stage > red ? stage : red;
}

template <int QT, int MT, int KW, bool F16OUT>
__global__ __launch_bounds__(64 * KW) void k_mmvq(const MmvqArgs args) {
  // per wave: this super-block's weight rows, batch rows and activation d;
  // after the K loop the same bytes hold the cross-wave partial tiles
  // (dynamic LDS: mmvq_lds_bytes<QT, MT, KW>() bytes, above the 64 KB static limit for KW = 8)
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  WaveLds<QT, MT> *lds = reinterpret_cast<WaveLds<QT, MT> *>(smem);
  f32x4(*red)[MT][64] = reinterpret_cast<f32x4(*)[MT][64]>(smem);

  const int bx = blockIdx.x;
  const int si = (args.nseg > 2 && bx >= args.seg[2].blk_begin) ? 2
                 : (args.nseg > 1 && bx >= args.seg[1].blk_begin) ? 1 : 0;
  const MmvqSeg &sg = args.seg[si];
  const int N = sg.N, M = args.M, K = args.K;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int l16 = lane & 15, q = lane >> 4;
  const int n0 = (bx - sg.blk_begin) * 16;
  const int nblk = K >> 5;
  const int nsb = (nblk + 7) >> 3;
  const uint32_t w_row = (QT == kTypeQ4_K)   ? static_cast<uint32_t>(K >> 8) * kQ4KBytes
                         : (QT == kTypeQ6_K) ? static_cast<uint32_t>(K >> 8) * kQ6KBytes
                                             : static_cast<uint32_t>(nblk) * kQ8_0Bytes;
  const uint32_t a_row = static_cast<uint32_t>(nblk) * kQ8_1Bytes;
  const rsrc_t Wr = make_rsrc(sg.W, w_row * static_cast<uint32_t>(N));
  const rsrc_t Ar = make_rsrc(args.A, a_row * static_cast<uint32_t>(M));
  bool a_ok[MT];
#pragma unroll
  for (int t = 0; t < MT; ++t) a_ok[t] = 16 * t + l16 < M;

  f32x4 acc[MT], accm[MT];
#pragma unroll
  for (int t = 0; t < MT; ++t) acc[t] = accm[t] = f32x4{0.f, 0.f, 0.f, 0.f};

  // Each super-block: 16-byte chunks (consecutive lanes on consecutive
  // bytes of a row) -> registers -> this wave's LDS slot -> MFMA operands.
  // The next super-block's chunks are in flight while this one is computed.
  WaveLds<QT, MT> &L = lds[wave];
  Chunks<QT, MT> ch;
  int sb = wave;
  if (sb < nsb) fetch<QT, MT>(ch, Wr, Ar, n0, N, M, w_row, a_row, sb, lane);
  for (; sb < nsb; sb += KW) {
    commit<QT, MT>(L, ch, M, lane);
    wave_sync();
    const bool more = sb + KW < nsb;
    if (more) fetch<QT, MT>(ch, Wr, Ar, n0, N, M, w_row, a_row, sb + KW, lane);
    WRegs<QT> wc;
    ARegs<MT> ac;
    read_w<QT, MT>(wc, L, l16, q, sb, nblk);
    read_a<QT, MT>(ac, L, a_ok, l16, q, sb, nblk);
    // activation d of batch rows 4q + i: through the dl table
#pragma unroll
    for (int t = 0; t < MT; ++t) {
      L.dl[t][q][l16] = h2f(ac.ds[t][0] & 0xFFFFu);
      L.dl[t][q + 4][l16] = h2f(ac.ds[t][1] & 0xFFFFu);
    }
    wave_sync();

    f32x4 P[MT];
#pragma unroll
    for (int t = 0; t < MT; ++t) P[t] = f32x4{0.f, 0.f, 0.f, 0.f};

    if constexpr (QT == kTypeQ4_K) {
      const uint32_t S0 = wc.hdr.y, S1 = wc.hdr.z, S2 = wc.hdr.w;
      // 6-bit scales / mins of sub-blocks 0-3 and 4-7 (quant_common.cuh:83-94)
      const uint64_t sc8 = static_cast<uint64_t>(S0 & 0x3F3F3F3Fu) |
                           (static_cast<uint64_t>((S2 & 0x0F0F0F0Fu) | ((S0 >> 2) & 0x30303030u)) << 32);
      const uint64_t mn8 = static_cast<uint64_t>(S1 & 0x3F3F3F3Fu) |
                           (static_cast<uint64_t>(((S2 >> 4) & 0x0F0F0F0Fu) | ((S1 >> 2) & 0x30303030u)) << 32);
#pragma unroll
    for (int b = 0; b < 8; ++b) {
        const u32x2 qq = wc.q[b >> 1];
        const int sh = (b & 1) * 4;
        const int64_t bw = pack64((qq.x >> sh) & 0x0F0F0F0Fu, (qq.y >> sh) & 0x0F0F0F0Fu);
        const int sc = static_cast<int>((sc8 >> (8 * b)) & 0xFFu);
#pragma unroll
        for (int t = 0; t < MT; ++t) {
          const i32x4 c = mfma_i8(ac.c[t][b], bw);
          const f32x4 d4 = *reinterpret_cast<const f32x4 *>(&L.dl[t][b][4 * q]);
#pragma unroll
          for (int i = 0; i < 4; ++i) P[t][i] += static_cast<float>(__mul24(c[i], sc)) * d4[i];
        }
      }
      const float d = h2f(wc.hdr.x & 0xFFFFu), dmin = h2f(wc.hdr.x >> 16);
      // min term: K = blocks 4j..4j+3 of a 16x16x4 fp32 MFMA; this lane
      // supplies block 4j + q of its batch row (s) and weight row (dmin*m)
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const float fm = dmin * static_cast<float>((mn8 >> (8 * (4 * j + q))) & 0xFFu);
#pragma unroll
        for (int t = 0; t < MT; ++t)
          accm[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(h2f(ac.ds[t][j] >> 16), fm, accm[t], 0, 0, 0);
      }
#pragma unroll
      for (int t = 0; t < MT; ++t) acc[t] += d * P[t];
    } else if constexpr (QT == kTypeQ6_K) {
      const bool first = q < 2;  // K chunks 0-15 of a block: scale 2*sub
#pragma unroll
      for (int b = 0; b < 8; ++b) {
        const int g = b >> 2, sub = b & 3;
        const u32x2 ql = wc.ql[2 * g + (sub & 1)];
        const u32x2 qh = wc.qh[g];
        const int lsh = (sub >= 2) ? 4 : 0, hsh = 2 * sub;
        const uint32_t v0 = q6_minus32(((ql.x >> lsh) & 0x0F0F0F0Fu) | (((qh.x >> hsh) & 0x03030303u) << 4));
        const uint32_t v1 = q6_minus32(((ql.y >> lsh) & 0x0F0F0F0Fu) | (((qh.y >> hsh) & 0x03030303u) << 4));
        const int64_t bw = pack64(v0, v1);
        const int64_t bw0 = first ? bw : 0, bw1 = first ? 0 : bw;
        const uint32_t scd = (b < 4) ? ((b < 2) ? wc.sc.x : wc.sc.y) : ((b < 6) ? wc.sc.z : wc.sc.w);
        const int sh = 16 * (b & 1);
        const int sc0 = static_cast<int8_t>((scd >> sh) & 0xFFu);
        const int sc1 = static_cast<int8_t>((scd >> (sh + 8)) & 0xFFu);
#pragma unroll
        for (int t = 0; t < MT; ++t) {
          const i32x4 c0 = mfma_i8(ac.c[t][b], bw0);
          const i32x4 c1 = mfma_i8(ac.c[t][b], bw1);
          const f32x4 d4 = *reinterpret_cast<const f32x4 *>(&L.dl[t][b][4 * q]);
#pragma unroll
          for (int i = 0; i < 4; ++i)
            P[t][i] += static_cast<float>(__mul24(c0[i], sc0) + __mul24(c1[i], sc1)) * d4[i];
        }
      }
      const float d = h2f(wc.d);
#pragma unroll
      for (int t = 0; t < MT; ++t) acc[t] += d * P[t];
    } else {
#pragma unroll
      for (int b = 0; b < 8; ++b) {
        const int64_t bw = pack64(wc.q[b].x, wc.q[b].y);
        const float dw = h2f(wc.d[b]);
#pragma unroll
        for (int t = 0; t < MT; ++t) {
          const i32x4 c = mfma_i8(ac.c[t][b], bw);
          const f32x4 d4 = *reinterpret_cast<const f32x4 *>(&L.dl[t][b][4 * q]);
#pragma unroll
          for (int i = 0; i < 4; ++i) P[t][i] += static_cast<float>(c[i]) * (dw * d4[i]);
        }
      }
#pragma unroll
      for (int t = 0; t < MT; ++t) acc[t] += P[t];
    }
    wave_sync();  // LDS reads of this super-block precede the next commit
  }
#pragma unroll
  for (int t = 0; t < MT; ++t) acc[t] -= accm[t];

  if constexpr (KW > 1) {
    __syncthreads();  // every wave is done with its staging slot
    if (wave > 0) {
#pragma unroll
      for (int t = 0; t < MT; ++t) red[wave - 1][t][lane] = acc[t];
    }
    __syncthreads();
    if (wave > 0) return;
#pragma unroll
    for (int w = 0; w < KW - 1; ++w)
#pragma unroll
      for (int t = 0; t < MT; ++t) acc[t] += red[w][t][lane];
  }

  // lane holds weight row n and batch rows 16t + 4q + i
  const int n = n0 + l16;
  if (n >= N) return;
  const int mode = args.mode;
#pragma unroll
  for (int t = 0; t < MT; ++t)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int m = 16 * t + 4 * q + i;
      if (m >= M) continue;
      const int64_t o = static_cast<int64_t>(m) * N + n;
      float y = acc[t][i];
      if constexpr (F16OUT) {
        uint16_t *Yh = static_cast<uint16_t *>(sg.Y);
        if (mode == kMvAccum) y += h2f(Yh[o]);
        else if (mode == kMvBias) y += h2f(static_cast<const uint16_t *>(sg.bias)[n]);
        Yh[o] = static_cast<uint16_t>(f2h_bits(y));
      } else {
        float *Yf = static_cast<float *>(sg.Y);
        if (mode == kMvAccum) y += Yf[o];
        else if (mode == kMvBias) y += static_cast<const float *>(sg.bias)[n];
        Yf[o] = y;
      }
    }
}

namespace {

// Waves per workgroup (K split): enough for ~2048 waves on the chip, at most
// eight and at most one per super-block.  IFX_MMVQ_KW in {1, 2, 4, 8}
// overrides (tuning; read once).
int choose_kw(int tiles, int nsb) {
  static const int env = [] {
    const char *e = ifx::tuning_env("IFX_MMVQ_KW");
    const int v = e ? atoi(e) : 0;
    return (v == 1 || v == 2 || v == 4 || v == 8) ? v : 0;
  }();
  int kw = env;
  if (!kw) {
    kw = 1;
    while (kw < 8 && tiles * kw < 2048) kw *= 2;
  }
  while (kw > 1 && kw > nsb) kw /= 2;
  return kw;
}

template <int QT, int MT, int KW, bool F16OUT>
void launch_one(const MmvqArgs &args, int blocks, hipStream_t s) {
  constexpr int lds = mmvq_lds_bytes<QT, MT, KW>();
  if constexpr (lds > 65536) {
    if (!dry_run()) {
      // once per instantiation: allow the dynamic LDS above 64 KB
      static const hipError_t attr = hipFuncSetAttribute(
          reinterpret_cast<const void *>(&k_mmvq<QT, MT, KW, F16OUT>),
          hipFuncAttributeMaxDynamicSharedMemorySize, lds);
      (void)attr;
    }
  }
  IFX_LAUNCH(k_mmvq, (QT, MT, KW, F16OUT), dim3(blocks), dim3(64 * KW), lds, s, args);
}

template <int QT, int MT, int KW>
void launch_kw(MmvqArgs args, int blocks, bool f16, hipStream_t s) {
  if (f16) launch_one<QT, MT, KW, true>(args, blocks, s);
  else launch_one<QT, MT, KW, false>(args, blocks, s);
}

template <int QT, int MT>
void launch_mt(MmvqArgs args, bool f16, hipStream_t s) {
  int blocks = 0;
  for (int i = 0; i < args.nseg; ++i) {
    args.seg[i].blk_begin = blocks;
    blocks += (args.seg[i].N + 15) / 16;
  }
  const int nsb = ((args.K >> 5) + 7) >> 3;
  switch (choose_kw(blocks, nsb)) {
  case 1: launch_kw<QT, MT, 1>(args, blocks, f16, s); break;
  case 2: launch_kw<QT, MT, 2>(args, blocks, f16, s); break;
  case 4: launch_kw<QT, MT, 4>(args, blocks, f16, s); break;
  default: launch_kw<QT, MT, 8>(args, blocks, f16, s); break;
  }
}

template <int QT>
void launch_q(const MmvqArgs &args, bool f16, hipStream_t s) {
  if (args.M <= 16) launch_mt<QT, 1>(args, f16, s);
  else launch_mt<QT, 2>(args, f16, s);
}

}  // namespace

// 1 <= M <= 32; K % 256 == 0 for Q4_K / Q6_K, K % 32 == 0 for Q8_0
// (checked by the caller).  count projections (1..3) share A.
hipError_t launch_mmvq(int qtype, int count, const void *const *W, void *const *Y,
                       const int *N, const void *bias, const void *A, bool f16, int M, int K,
                       int mode, hipStream_t stream) {
  if (M < 1 || M > 32 || count < 1 || count > 3) return hipErrorInvalidValue;
  MmvqArgs args{};
  for (int i = 0; i < count; ++i)
    args.seg[i] = MmvqSeg{static_cast<const uint8_t *>(W[i]), Y[i], i == 0 ? bias : nullptr, N[i], 0};
  args.nseg = count;
  args.A = static_cast<const uint8_t *>(A);
  args.M = M;
  args.K = K;
  args.mode = mode;
  switch (qtype) {
  case kTypeQ4_K: launch_q<kTypeQ4_K>(args, f16, stream); break;
  case kTypeQ6_K: launch_q<kTypeQ6_K>(args, f16, stream); break;
  case kTypeQ8_0: launch_q<kTypeQ8_0>(args, f16, stream); break;
  default: return hipErrorInvalidValue;
  }
  return last_error();
}

}  // namespace ifx
