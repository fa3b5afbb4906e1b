// gemm_mfma.hip -- int8-MFMA GEMM for prefill and large decode batches
// (M > 32) on gfx950: y[m][n] = sum_k W[n][k] * a[m][k], W raw GGUF Q4_K /
// Q6_K / Q8_0 blocks, a Q8_1 blocks of 32, fp32 accumulate.
//
// The reference has no quantized GEMM above M = 64: it dequantizes W to
// FP16 and calls cuBLAS (runtime/backends/cuda/native/
// quantized_weight_map.cpp:176-233, cublas_gemm.h:47; caller
// transformer_forward.cu:1479), and its MMQ kernels for 9 <= M <= 64
// (kernels/mmq.cuh:41-835) use dp4a.  This kernel keeps the MMQ arithmetic
// of the GEMV path -- an exact integer dot per 32-value block (16-value
// group for Q6_K), then fp32 scaling by the weight and activation block
// scales -- with the integer dot on the matrix cores.
//
// Tiling: a 256-thread workgroup owns a 128 (m) x 128 (n) output tile (64 x
// 64 when that gives fewer than two workgroups per CU); its four waves are
// 2 x 2, each owning 2 x 2 (or one) MFMA tiles of 32 x 32.
// The K loop steps one 256-value super-block at a time:
//   1. the next super-block's A items (Q8_1 blocks of 128 rows) and raw W
//      bytes (16-byte chunks of 128 rows) are loaded into registers while
//      the current one is computed; at the top of a step they are written
//      to LDS (about 61 KB for Q4_K: two workgroups per CU);
//   2. each wave unpacks W codes to int8 MFMA operands from LDS (Q4_K
//      nibbles; Q6_K 4+2 bits minus 32; Q8_0 as is) and runs
//      v_mfma_i32_32x32x32_i8 per 32-value block (two
//      v_mfma_i32_32x32x16_i8 for Q6_K, whose scales are per 16 values);
//   3. the int32 block results are scaled into fp32 accumulators with
//      three VALU operations per output (scale product, convert, FMA):
//      Q4_K  acc += C * (da * d*sc) - sa * (dmin*m)          (mmvq.cuh:115-125)
//      Q6_K  acc += (sc0*C0 + sc1*C1) * (da * d)             (mmvq.cuh:467-471)
//      Q8_0  acc += C * (da * dw)                            (mmvq.cuh:886-889)
//      The Q4_K min term is an fp32 GEMM over the 8 sub-blocks of a
//      super-block, run on the matrix cores (v_mfma_f32_32x32x2f32) into
//      the same accumulators, so it costs no VALU time.
// This per-block rescaling (the activation d varies per row and per 32
// values, the weight scale per column and per 32 values) is VALU work the
// matrix cores cannot absorb: at three operations per output per block it
// bounds the kernel near 15 % of the int8 MFMA peak.
// MFMA lane layouts (32x32 output): lane l supplies row (l % 32) of A and
// column (l % 32) of B for the K half (l / 32); it receives column l % 32
// and rows 8*(i/4) + 4*(l/32) + (i%4), i = 0..15, of the result.
#include "ifx_common.h"

namespace ifx {

namespace {

constexpr int kApitch = 256 + 16;  // int8 codes per staged A row (+pad vs bank conflicts)

template <int QT>
struct GFmt;
template <>
struct GFmt<kTypeQ4_K> {  // raw super-block per row: 9 chunks of 16 bytes
  static constexpr int kSb = 144, kPitch = 144 + 16, kChunks = 9;
};
template <>
struct GFmt<kTypeQ6_K> {  // 210 bytes; the 14th chunk carries only d
  static constexpr int kSb = 210, kPitch = 224 + 16, kChunks = 14;
};
template <>
struct GFmt<kTypeQ8_0> {  // codes of 8 blocks [row][b*32], d separately
  static constexpr int kSb = 272, kPitch = 256 + 16, kChunks = 0;
};

// Workgroup tile: 64*S x 64*S (m x n); each of the 2 x 2 waves owns S x S
// MFMA tiles of 32 x 32.
template <int QT, int S>
struct Smem {
  static constexpr int kBM = 64 * S, kBN = 64 * S;
  int8_t a[kBM * kApitch];             // activation codes [m][k within super-block]
  float da[8][kBM];                    // Q8_1 d per block, [block][m]
  float sa[8][kBM];                    // Q8_1 s per block, [block][m]
  uint8_t w[kBN * GFmt<QT>::kPitch];   // raw W super-block per row (Q8_0: codes)
  float dw[QT == kTypeQ8_0 ? 8 : 1][kBN];  // Q8_0 per-block weight d
};

// One super-block of the workgroup's tile in a thread's registers.
template <int QT, int S>
struct Prefetch {
  static constexpr int kBM = 64 * S, kBN = 64 * S;
  static constexpr int kAItems = kBM * 8 / 256;  // (row, block) items per thread
  static constexpr int kWItems =
      QT == kTypeQ8_0 ? kBN * 8 / 256 : (kBN * GFmt<QT>::kChunks + 255) / 256;
  uint32_t ads[kAItems];
  i32x4 a0[kAItems], a1[kAItems];
  u32x4 w0[kWItems];
  u32x4 w1[QT == kTypeQ8_0 ? kWItems : 1];  // Q8_0: codes 16-31
  uint32_t wd[QT == kTypeQ8_0 ? kWItems : 1];
};

__device__ __forceinline__ i32x16 mfma32(i32x4 a, i32x4 b) {
  const i32x16 z = {0};
  return __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, z, 0, 0, 0);
}

__device__ __forceinline__ i32x16 mfma16(int64_t a, int64_t b) {
  const i32x16 z = {0};
  return __builtin_amdgcn_mfma_i32_32x32x16_i8(a, b, z, 0, 0, 0);
}

// Q6_K code bytes v in [0, 63] -> int8 (v - 32), four per dword, no carries:
// flip bit 5, then sign-extend the new bit 5 into bits 6 and 7.
__device__ __forceinline__ uint32_t q6_minus32(uint32_t v) {
  uint32_t x = v ^ 0x20202020u;
  const uint32_t t = x & 0x20202020u;
  return x | (t << 1) | (t << 2);
}

template <int QT, int S>
__device__ __forceinline__ void fetch(Prefetch<QT, S> &pf, rsrc_t Wr, rsrc_t Ar, uint32_t w_row,
                                      uint32_t a_row, int m0, int n0, int M, int N, int sblk,
                                      int tid) {
  constexpr int kBN = Prefetch<QT, S>::kBN;
#pragma unroll
  for (int i = 0; i < Prefetch<QT, S>::kAItems; ++i) {
    const int it = tid + 256 * i;
    const int r = it >> 3, b = it & 7;
    pf.ads[i] = 0;
    pf.a0[i] = pf.a1[i] = i32x4{0, 0, 0, 0};
    if (m0 + r < M) {
      const uint32_t o = (m0 + r) * a_row + (sblk * 8 + b) * kQ8_1Bytes;
      pf.ads[i] = bload<uint32_t>(Ar, o, 0);
      pf.a0[i] = bload<i32x4>(Ar, o + 4, 0);
      pf.a1[i] = bload<i32x4>(Ar, o + 20, 0);
    }
  }
  using F = GFmt<QT>;
  if constexpr (QT == kTypeQ8_0) {
#pragma unroll
    for (int i = 0; i < Prefetch<QT, S>::kWItems; ++i) {
      const int it = tid + 256 * i;
      const int r = it >> 3, b = it & 7;
      const uint32_t o = min(n0 + r, N - 1) * w_row + (sblk * 8 + b) * kQ8_0Bytes;
      pf.wd[i] = wload<uint16_t>(Wr, o, 0);
      pf.w0[i] = wload<u32x4>(Wr, o + 2, 0);
      pf.w1[i] = wload<u32x4>(Wr, o + 18, 0);
    }
  } else {
#pragma unroll
    for (int i = 0; i < Prefetch<QT, S>::kWItems; ++i) {
      const int c = tid + 256 * i;
      pf.w0[i] = u32x4{0, 0, 0, 0};
      if (c < kBN * F::kChunks) {
        const int r = c / F::kChunks, part = c - r * F::kChunks;
        const uint32_t o = min(n0 + r, N - 1) * w_row + sblk * F::kSb + 16 * part;
        // the last Q6_K chunk holds only d: a 16-byte load could cross the
        // end of the tensor on its last super-block (and then read zeros)
        if (QT == kTypeQ6_K && part == 13) pf.w0[i].x = wload<uint16_t>(Wr, o, 0);
        else pf.w0[i] = wload<u32x4>(Wr, o, 0);
      }
    }
  }
}

template <int QT, int S>
__device__ __forceinline__ void commit(Smem<QT, S> &sm, const Prefetch<QT, S> &pf, int tid) {
  constexpr int kBN = Prefetch<QT, S>::kBN;
#pragma unroll
  for (int i = 0; i < Prefetch<QT, S>::kAItems; ++i) {
    const int it = tid + 256 * i;
    const int r = it >> 3, b = it & 7;
    *reinterpret_cast<i32x4 *>(&sm.a[r * kApitch + b * 32]) = pf.a0[i];
    *reinterpret_cast<i32x4 *>(&sm.a[r * kApitch + b * 32 + 16]) = pf.a1[i];
    sm.da[b][r] = h2f(pf.ads[i] & 0xFFFFu);
    sm.sa[b][r] = h2f(pf.ads[i] >> 16);
  }
  using F = GFmt<QT>;
  if constexpr (QT == kTypeQ8_0) {
#pragma unroll
    for (int i = 0; i < Prefetch<QT, S>::kWItems; ++i) {
      const int it = tid + 256 * i;
      const int r = it >> 3, b = it & 7;
      *reinterpret_cast<u32x4 *>(&sm.w[r * F::kPitch + b * 32]) = pf.w0[i];
      *reinterpret_cast<u32x4 *>(&sm.w[r * F::kPitch + b * 32 + 16]) = pf.w1[i];
      sm.dw[b][r] = h2f(pf.wd[i]);
    }
  } else {
#pragma unroll
    for (int i = 0; i < Prefetch<QT, S>::kWItems; ++i) {
      const int c = tid + 256 * i;
      if (c < kBN * F::kChunks) {
        const int r = c / F::kChunks, part = c - r * F::kChunks;
        *reinterpret_cast<u32x4 *>(&sm.w[r * F::kPitch + 16 * part]) = pf.w0[i];
      }
    }
  }
}

}  // namespace

template <int QT, int S, bool F16OUT>
__global__ __launch_bounds__(256, 2) void k_gemm_mfma(const uint8_t *__restrict__ W,
                                                      const uint8_t *__restrict__ A,
                                                      void *__restrict__ Y,
                                                      const void *__restrict__ bias, int M,
                                                      int N, int K, int mode) {
  using F = GFmt<QT>;
  extern __shared__ __attribute__((aligned(16))) uint8_t smem_raw[];
  Smem<QT, S> &sm = *reinterpret_cast<Smem<QT, S> *>(smem_raw);
  constexpr int kBM = 64 * S, kBN = 64 * S;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave & 1, wn = wave >> 1;  // wave position in the 2 x 2 grid
  const int m0 = blockIdx.y * kBM, n0 = blockIdx.x * kBN;
  const int l32 = lane & 31, h = lane >> 5;
  const int nblk32 = K >> 5;
  const uint32_t a_row = static_cast<uint32_t>(nblk32) * kQ8_1Bytes;
  const uint32_t w_row = static_cast<uint32_t>(QT == kTypeQ8_0 ? nblk32 * kQ8_0Bytes
                                                               : (K >> 8) * F::kSb);
  const rsrc_t Wr = make_rsrc(W, w_row * static_cast<uint32_t>(N));
  const rsrc_t Ar = make_rsrc(A, a_row * static_cast<uint32_t>(M));

  f32x16 acc[S][S];
#pragma unroll
  for (int a = 0; a < S; ++a)
#pragma unroll
    for (int b = 0; b < S; ++b)
#pragma unroll
      for (int i = 0; i < 16; ++i) acc[a][b][i] = 0.0f;

  // Rows of this wave's A tiles and columns of its B tiles; first of the 4
  // consecutive result rows this lane holds per group of 4.
  int ar[S], bn[S], rbase[S];
#pragma unroll
  for (int j = 0; j < S; ++j) {
    ar[j] = wm * 32 * S + 32 * j + l32;
    bn[j] = wn * 32 * S + 32 * j + l32;
    rbase[j] = wm * 32 * S + 32 * j + 4 * h;
  }

  const int nsteps = K >> 8;
  Prefetch<QT, S> pf;
  fetch<QT, S>(pf, Wr, Ar, w_row, a_row, m0, n0, M, N, 0, tid);
  for (int sblk = 0; sblk < nsteps; ++sblk) {
    __syncthreads();  // previous step's LDS reads are done
    commit<QT, S>(sm, pf, tid);
    __syncthreads();
    if (sblk + 1 < nsteps) fetch<QT, S>(pf, Wr, Ar, w_row, a_row, m0, n0, M, N, sblk + 1, tid);

    if constexpr (QT == kTypeQ4_K) {
      float dsc[S][8];
#pragma unroll
      for (int t = 0; t < S; ++t) {
        const u32x4 hdr = *reinterpret_cast<const u32x4 *>(&sm.w[bn[t] * F::kPitch]);
        const float d = h2f(hdr.x & 0xFFFFu), dmin = h2f(hdr.x >> 16);
        const uint32_t S0 = hdr.y, S1 = hdr.z, S2 = hdr.w;
        const uint32_t sc_lo = S0 & 0x3F3F3F3Fu, m_lo = S1 & 0x3F3F3F3Fu;
        const uint32_t sc_hi = (S2 & 0x0F0F0F0Fu) | ((S0 >> 2) & 0x30303030u);
        const uint32_t m_hi = ((S2 >> 4) & 0x0F0F0F0Fu) | ((S1 >> 2) & 0x30303030u);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          dsc[t][j] = d * static_cast<float>((sc_lo >> (8 * j)) & 0xFFu);
          dsc[t][j + 4] = d * static_cast<float>((sc_hi >> (8 * j)) & 0xFFu);
        }
        // min term on the matrix cores, subtracted straight from the
        // accumulators: K = sub-blocks 2j + h, j = 0..3
        const uint64_t mm = static_cast<uint64_t>(m_lo) | (static_cast<uint64_t>(m_hi) << 32);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int blk = 2 * j + h;
          const float fm = -(dmin * static_cast<float>((mm >> (8 * blk)) & 0xFFu));
#pragma unroll
          for (int s = 0; s < S; ++s)
            acc[s][t] = __builtin_amdgcn_mfma_f32_32x32x2f32(sm.sa[blk][ar[s]], fm, acc[s][t],
                                                             0, 0, 0);
        }
      }
#pragma unroll
      for (int p = 0; p < 4; ++p) {
        // Sub-blocks 2p (low nibbles) and 2p+1 (high nibbles) share qs bytes.
        u32x4 q[S];
#pragma unroll
        for (int t = 0; t < S; ++t)
          q[t] = *reinterpret_cast<const u32x4 *>(&sm.w[bn[t] * F::kPitch + 16 + p * 32 + 16 * h]);
#pragma unroll
        for (int half = 0; half < 2; ++half) {
          const int sb = 2 * p + half;
          const int sh = 4 * half;
          i32x4 bw[S], av[S];
#pragma unroll
          for (int t = 0; t < S; ++t)
            bw[t] = i32x4{static_cast<int>((q[t].x >> sh) & 0x0F0F0F0Fu),
                          static_cast<int>((q[t].y >> sh) & 0x0F0F0F0Fu),
                          static_cast<int>((q[t].z >> sh) & 0x0F0F0F0Fu),
                          static_cast<int>((q[t].w >> sh) & 0x0F0F0F0Fu)};
#pragma unroll
          for (int s = 0; s < S; ++s)
            av[s] = *reinterpret_cast<const i32x4 *>(&sm.a[ar[s] * kApitch + sb * 32 + 16 * h]);
#pragma unroll
          for (int s = 0; s < S; ++s) {
            f32x4 fa[4];
#pragma unroll
            for (int g = 0; g < 4; ++g)
              fa[g] = *reinterpret_cast<const f32x4 *>(&sm.da[sb][rbase[s] + 8 * g]);
#pragma unroll
            for (int t = 0; t < S; ++t) {
              const i32x16 c = mfma32(av[s], bw[t]);
              const float w = dsc[t][sb];
#pragma unroll
              for (int i = 0; i < 16; ++i)
                acc[s][t][i] += static_cast<float>(c[i]) * (fa[i >> 2][i & 3] * w);
            }
          }
        }
      }
    } else if constexpr (QT == kTypeQ6_K) {
      float dq[S];
      uint32_t scw[S][4];
#pragma unroll
      for (int t = 0; t < S; ++t) {
        const uint8_t *row = &sm.w[bn[t] * F::kPitch];
        dq[t] = h2f(*reinterpret_cast<const uint16_t *>(row + 208));
        const u32x4 s4 = *reinterpret_cast<const u32x4 *>(row + 192);
        scw[t][0] = s4.x; scw[t][1] = s4.y; scw[t][2] = s4.z; scw[t][3] = s4.w;
      }
#pragma unroll
      for (int g = 0; g < 2; ++g) {
#pragma unroll
        for (int sub = 0; sub < 4; ++sub) {
          const int sb = g * 4 + sub;  // Q8_1 block within the super-block
          // 16-value group u (0/1): values 16u..16u+15 of this 32-run; this
          // lane supplies values 16u + 8h .. 16u + 8h + 7.
          int64_t bq[S][2];
          int s0[S], s1[S];
#pragma unroll
          for (int t = 0; t < S; ++t) {
            const uint8_t *row = &sm.w[bn[t] * F::kPitch];
#pragma unroll
            for (int u = 0; u < 2; ++u) {
              const int e = 16 * u + 8 * h;
              const u32x2 ql = *reinterpret_cast<const u32x2 *>(row + g * 64 + (sub & 1) * 32 + e);
              const u32x2 qh = *reinterpret_cast<const u32x2 *>(row + 128 + g * 32 + e);
              const int lsh = (sub >= 2) ? 4 : 0, hsh = 2 * sub;
              const uint32_t v0 = ((ql.x >> lsh) & 0x0F0F0F0Fu) | (((qh.x >> hsh) & 0x03030303u) << 4);
              const uint32_t v1 = ((ql.y >> lsh) & 0x0F0F0F0Fu) | (((qh.y >> hsh) & 0x03030303u) << 4);
              bq[t][u] = static_cast<int64_t>(q6_minus32(v0)) |
                         (static_cast<int64_t>(q6_minus32(v1)) << 32);
            }
            // scales[g*8 + 2*sub + u]
            const uint32_t sw = scw[t][2 * g + (sub >> 1)] >> (16 * (sub & 1));
            s0[t] = static_cast<int8_t>(sw & 0xFFu);
            s1[t] = static_cast<int8_t>((sw >> 8) & 0xFFu);
          }
#pragma unroll
          for (int s = 0; s < S; ++s) {
            int64_t aq[2];
#pragma unroll
            for (int u = 0; u < 2; ++u)
              aq[u] = *reinterpret_cast<const int64_t *>(&sm.a[ar[s] * kApitch + sb * 32 + 16 * u + 8 * h]);
            f32x4 fa[4];
#pragma unroll
            for (int gg = 0; gg < 4; ++gg)
              fa[gg] = *reinterpret_cast<const f32x4 *>(&sm.da[sb][rbase[s] + 8 * gg]);
#pragma unroll
            for (int t = 0; t < S; ++t) {
              const i32x16 c0 = mfma16(aq[0], bq[t][0]);
              const i32x16 c1 = mfma16(aq[1], bq[t][1]);
              const float dd = dq[t];
#pragma unroll
              for (int i = 0; i < 16; ++i) {
                const int ci = __mul24(c0[i], s0[t]) + __mul24(c1[i], s1[t]);
                acc[s][t][i] += static_cast<float>(ci) * (fa[i >> 2][i & 3] * dd);
              }
            }
          }
        }
      }
    } else {
#pragma unroll
      for (int b = 0; b < 8; ++b) {
        i32x4 bw[S];
        float dwv[S];
#pragma unroll
        for (int t = 0; t < S; ++t) {
          bw[t] = *reinterpret_cast<const i32x4 *>(&sm.w[bn[t] * F::kPitch + b * 32 + 16 * h]);
          dwv[t] = sm.dw[b][bn[t]];
        }
#pragma unroll
        for (int s = 0; s < S; ++s) {
          const i32x4 av = *reinterpret_cast<const i32x4 *>(&sm.a[ar[s] * kApitch + b * 32 + 16 * h]);
          f32x4 fa[4];
#pragma unroll
          for (int gg = 0; gg < 4; ++gg)
            fa[gg] = *reinterpret_cast<const f32x4 *>(&sm.da[b][rbase[s] + 8 * gg]);
#pragma unroll
          for (int t = 0; t < S; ++t) {
            const i32x16 c = mfma32(av, bw[t]);
#pragma unroll
            for (int i = 0; i < 16; ++i)
              acc[s][t][i] += static_cast<float>(c[i]) * (fa[i >> 2][i & 3] * dwv[t]);
          }
        }
      }
    }
  }

  // Epilogue: lane holds column n and rows rbase + 8g + j.
#pragma unroll
  for (int s = 0; s < S; ++s)
#pragma unroll
    for (int t = 0; t < S; ++t) {
      const int n = n0 + wn * 32 * S + 32 * t + l32;
      if (n >= N) continue;
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int m = m0 + wm * 32 * S + 32 * s + 8 * (i >> 2) + 4 * h + (i & 3);
        if (m >= M) continue;
        const int64_t o = static_cast<int64_t>(m) * N + n;
        float y = acc[s][t][i];
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

template <int QT, int S>
static hipError_t launch_qts(const uint8_t *W, const uint8_t *A, void *Y, const void *bias,
                             bool f16, int M, int N, int K, int mode, hipStream_t s) {
  constexpr int kB = 64 * S;
  const dim3 grid((N + kB - 1) / kB, (M + kB - 1) / kB);
  const size_t shm = sizeof(Smem<QT, S>);
  // The staged tiles can exceed the 64 KiB default; gfx950 has 160 KiB of LDS.
  // set once per kernel (function-local statics: thread-safe)
  if (!dry_run()) {
    static const hipError_t attr_f32 = hipFuncSetAttribute(
        reinterpret_cast<const void *>(&k_gemm_mfma<QT, S, false>),
        hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(shm));
    static const hipError_t attr_f16 = hipFuncSetAttribute(
        reinterpret_cast<const void *>(&k_gemm_mfma<QT, S, true>),
        hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(shm));
    const hipError_t attr = f16 ? attr_f16 : attr_f32;
    if (attr != hipSuccess) return attr;
  }
  if (f16)
    IFX_LAUNCH(k_gemm_mfma, (QT, S, true), grid, dim3(256), shm, s, W, A, Y, bias, M, N, K, mode);
  else
    IFX_LAUNCH(k_gemm_mfma, (QT, S, false), grid, dim3(256), shm, s, W, A, Y, bias, M, N, K, mode);
  return last_error();
}

// 128 x 128 workgroup tiles when they give at least two workgroups per CU,
// else 64 x 64 (e.g. N = 5120 at M = 512: 160 large tiles, 640 small).
template <int QT>
static hipError_t launch_qt(const uint8_t *W, const uint8_t *A, void *Y, const void *bias, bool f16,
                            int M, int N, int K, int mode, hipStream_t s) {
  const int64_t big = static_cast<int64_t>((N + 127) / 128) * ((M + 127) / 128);
  if (big >= 512) return launch_qts<QT, 2>(W, A, Y, bias, f16, M, N, K, mode, s);
  return launch_qts<QT, 1>(W, A, Y, bias, f16, M, N, K, mode, s);
}

hipError_t launch_gemv(int qtype, const void *W, const void *A, void *Y, const void *bias,
                       bool f16, int M, int N, int K, int mode, hipStream_t stream);

// K % 256 == 0 is required for the super-block K loop; Q8_0 weights with
// K % 256 != 0 run on the GEMV kernel in groups of 8 columns instead.
hipError_t launch_gemm_mfma(int qtype, const void *W, const void *A, void *Y, const void *bias,
                            bool f16, int M, int N, int K, int mode, hipStream_t stream) {
  const uint8_t *w = static_cast<const uint8_t *>(W);
  const uint8_t *a = static_cast<const uint8_t *>(A);
  if (K % 256 != 0) return launch_gemv(qtype, W, A, Y, bias, f16, M, N, K, mode, stream);
  switch (qtype) {
  case kTypeQ4_K: return launch_qt<kTypeQ4_K>(w, a, Y, bias, f16, M, N, K, mode, stream);
  case kTypeQ6_K: return launch_qt<kTypeQ6_K>(w, a, Y, bias, f16, M, N, K, mode, stream);
  case kTypeQ8_0: return launch_qt<kTypeQ8_0>(w, a, Y, bias, f16, M, N, K, mode, stream);
  default: return hipErrorInvalidValue;
  }
}

}  // namespace ifx
