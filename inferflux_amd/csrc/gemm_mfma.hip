// gemm_mfma.hip -- int8-MFMA GEMM for prefill and large decode batches
// (M > 8) on gfx950: y[m][n] = sum_k W[n][k] * a[m][k], W raw GGUF Q4_K /
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
// Tiling: a 256-thread workgroup owns a 128 (m) x 128 (n) output tile; its
// four waves are 2 x 2, each owning 64 x 64 = 2 x 2 MFMA tiles of 32 x 32.
// The K loop steps one 256-value super-block at a time:
//   1. the workgroup stages A (128 rows x 8 Q8_1 blocks: codes + fp32 d and
//      s) and the raw W super-blocks of its 128 rows in LDS;
//   2. each wave unpacks W codes to int8 MFMA operands straight from LDS
//      (Q4_K nibbles; Q6_K 4+2 bits minus 32; Q8_0 as is) and runs
//      v_mfma_i32_32x32x32_i8 per 32-value block (two
//      v_mfma_i32_32x32x16_i8 for Q6_K, whose scales are per 16 values);
//   3. the int32 block results are scaled into fp32 accumulators:
//      Q4_K  acc += (d*sc) * da * C - (dmin*m) * sa      (mmvq.cuh:115-125)
//      Q6_K  acc += d * da * (sc0*C0 + sc1*C1)           (mmvq.cuh:467-471)
//      Q8_0  acc += dw * da * C                          (mmvq.cuh:886-889)
// MFMA lane layouts (32x32 output): lane l supplies row (l % 32) of A and
// column (l % 32) of B for the K half (l / 32); it receives column l % 32
// and rows 8*(i/4) + 4*(l/32) + (i%4), i = 0..15, of the result.
#include "ifx_common.h"

namespace ifx {

namespace {

constexpr int kBM = 128, kBN = 128;
constexpr int kApitch = 256 + 16;  // int8 codes per staged A row (+pad vs bank conflicts)
constexpr int kWpitch = 256 + 16;  // staged W bytes per row: raw Q4_K/Q6_K block or 8 Q8_0 code runs

typedef int32_t i32x2 __attribute__((ext_vector_type(2)));

struct Smem {
  int8_t a[kBM * kApitch];  // activation codes [m][k within super-block]
  float da[8][kBM];         // Q8_1 d per block, [block][m]
  float sa[8][kBM];         // Q8_1 s per block, [block][m]
  uint8_t w[kBN * kWpitch]; // raw W super-block per row (Q8_0: codes, see below)
  float dw[8][kBN];         // Q8_0 per-block weight scale
};

__device__ __forceinline__ i32x16 mfma32(i32x4 a, i32x4 b, i32x16 c) {
  return __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ i32x16 mfma16(int64_t a, int64_t b, i32x16 c) {
  return __builtin_amdgcn_mfma_i32_32x32x16_i8(a, b, c, 0, 0, 0);
}

// Q6_K code bytes v in [0, 63] -> int8 (v - 32), four per dword, no carries:
// flip bit 5, then sign-extend the new bit 5 into bits 6 and 7.
__device__ __forceinline__ uint32_t q6_minus32(uint32_t v) {
  uint32_t x = v ^ 0x20202020u;
  const uint32_t t = x & 0x20202020u;
  return x | (t << 1) | (t << 2);
}

template <int QT>
__device__ __forceinline__ void stage(Smem &sm, const uint8_t *__restrict__ W,
                                      const uint8_t *__restrict__ A, int m0, int n0, int M, int N,
                                      int K, int sblk, int tid) {
  const int nblk32 = K >> 5;
  // A: 128 rows x 8 blocks; one (row, block) item per thread per pass.
  for (int it = tid; it < kBM * 8; it += 256) {
    const int r = it >> 3, b = it & 7;
    const int m = m0 + r;
    i32x4 c0 = {0, 0, 0, 0}, c1 = {0, 0, 0, 0};
    uint32_t ds = 0;
    if (m < M) {
      const uint8_t *src = A + (static_cast<int64_t>(m) * nblk32 + sblk * 8 + b) * kQ8_1Bytes;
      ds = ldg<uint32_t>(src);
      c0 = ldg<i32x4>(src + 4);
      c1 = ldg<i32x4>(src + 20);
    }
    *reinterpret_cast<i32x4 *>(&sm.a[r * kApitch + b * 32]) = c0;
    *reinterpret_cast<i32x4 *>(&sm.a[r * kApitch + b * 32 + 16]) = c1;
    sm.da[b][r] = h2f(ds & 0xFFFFu);
    sm.sa[b][r] = h2f(ds >> 16);
  }
  if constexpr (QT == kTypeQ4_K) {
    const int nsb = K >> 8;
    for (int it = tid; it < kBN * 9; it += 256) {
      const int r = it / 9, c = it - r * 9;
      const int n = n0 + r;
      u32x4 v = {0, 0, 0, 0};
      if (n < N) v = ldg<u32x4>(W + (static_cast<int64_t>(n) * nsb + sblk) * kQ4KBytes + c * 16);
      *reinterpret_cast<u32x4 *>(&sm.w[r * kWpitch + c * 16]) = v;
    }
  } else if constexpr (QT == kTypeQ6_K) {
    const int nsb = K >> 8;
    for (int it = tid; it < kBN * 14; it += 256) {
      const int r = it / 14, c = it - r * 14;
      const int n = n0 + r;
      u32x4 v = {0, 0, 0, 0};
      if (n < N) {
        const uint8_t *src = W + (static_cast<int64_t>(n) * nsb + sblk) * kQ6KBytes + c * 16;
        if (c < 13) v = ldg<u32x4>(src);
        else v.x = ldg<uint16_t>(src);  // bytes 208-209: d; never read past the block
      }
      *reinterpret_cast<u32x4 *>(&sm.w[r * kWpitch + c * 16]) = v;
    }
  } else {
    // Q8_0: 8 blocks of 34 B per row and step; codes to [row][b*32], d to dw.
    for (int it = tid; it < kBN * 8; it += 256) {
      const int r = it >> 3, b = it & 7;
      const int n = n0 + r;
      i32x4 c0 = {0, 0, 0, 0}, c1 = {0, 0, 0, 0};
      float d = 0.0f;
      if (n < N) {
        const uint8_t *src = W + (static_cast<int64_t>(n) * nblk32 + sblk * 8 + b) * kQ8_0Bytes;
        d = h2f(ldg<uint16_t>(src));
        c0 = ldg<i32x4>(src + 2);
        c1 = ldg<i32x4>(src + 18);
      }
      *reinterpret_cast<i32x4 *>(&sm.w[r * kWpitch + b * 32]) = c0;
      *reinterpret_cast<i32x4 *>(&sm.w[r * kWpitch + b * 32 + 16]) = c1;
      sm.dw[b][r] = d;
    }
  }
}

}  // namespace

template <int QT, bool F16OUT>
__global__ __launch_bounds__(256) void k_gemm_mfma(const uint8_t *__restrict__ W,
                                                   const uint8_t *__restrict__ A,
                                                   void *__restrict__ Y,
                                                   const void *__restrict__ bias, int M, int N,
                                                   int K, int mode) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem_raw[];
  Smem &sm = *reinterpret_cast<Smem *>(smem_raw);
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave & 1, wn = wave >> 1;  // wave position in the 2 x 2 grid
  const int m0 = blockIdx.y * kBM, n0 = blockIdx.x * kBN;
  const int l32 = lane & 31, h = lane >> 5;

  f32x16 acc[2][2];
#pragma unroll
  for (int a = 0; a < 2; ++a)
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
      for (int i = 0; i < 16; ++i) acc[a][b][i] = 0.0f;

  const int nsteps = K >> 8;
  for (int sblk = 0; sblk < nsteps; ++sblk) {
    __syncthreads();  // previous step's LDS reads are done
    stage<QT>(sm, W, A, m0, n0, M, N, K, sblk, tid);
    __syncthreads();

    // Rows of this wave's A tiles and columns of its B tiles.
    const int ar[2] = {wm * 64 + l32, wm * 64 + 32 + l32};
    const int bn[2] = {wn * 64 + l32, wn * 64 + 32 + l32};
    // First of the 4 consecutive result rows this lane holds per group of 4.
    const int rbase[2] = {wm * 64 + 4 * h, wm * 64 + 32 + 4 * h};

    if constexpr (QT == kTypeQ4_K) {
      float fw[2][8], fm[2][8];
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const u32x4 hdr = *reinterpret_cast<const u32x4 *>(&sm.w[bn[t] * kWpitch]);
        const float d = h2f(hdr.x & 0xFFFFu), dmin = h2f(hdr.x >> 16);
        const uint32_t S0 = hdr.y, S1 = hdr.z, S2 = hdr.w;
        const uint32_t sc_lo = S0 & 0x3F3F3F3Fu, m_lo = S1 & 0x3F3F3F3Fu;
        const uint32_t sc_hi = (S2 & 0x0F0F0F0Fu) | ((S0 >> 2) & 0x30303030u);
        const uint32_t m_hi = ((S2 >> 4) & 0x0F0F0F0Fu) | ((S1 >> 2) & 0x30303030u);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          fw[t][j] = d * static_cast<float>((sc_lo >> (8 * j)) & 0xFFu);
          fw[t][j + 4] = d * static_cast<float>((sc_hi >> (8 * j)) & 0xFFu);
          fm[t][j] = dmin * static_cast<float>((m_lo >> (8 * j)) & 0xFFu);
          fm[t][j + 4] = dmin * static_cast<float>((m_hi >> (8 * j)) & 0xFFu);
        }
      }
#pragma unroll
      for (int p = 0; p < 4; ++p) {
        // Sub-blocks 2p (low nibbles) and 2p+1 (high nibbles) share qs bytes.
        i32x4 blo[2], bhi[2];
#pragma unroll
        for (int t = 0; t < 2; ++t) {
          const u32x4 q =
              *reinterpret_cast<const u32x4 *>(&sm.w[bn[t] * kWpitch + 16 + p * 32 + 16 * h]);
          blo[t] = i32x4{static_cast<int>(q.x & 0x0F0F0F0Fu), static_cast<int>(q.y & 0x0F0F0F0Fu),
                         static_cast<int>(q.z & 0x0F0F0F0Fu), static_cast<int>(q.w & 0x0F0F0F0Fu)};
          bhi[t] = i32x4{static_cast<int>((q.x >> 4) & 0x0F0F0F0Fu),
                         static_cast<int>((q.y >> 4) & 0x0F0F0F0Fu),
                         static_cast<int>((q.z >> 4) & 0x0F0F0F0Fu),
                         static_cast<int>((q.w >> 4) & 0x0F0F0F0Fu)};
        }
#pragma unroll
        for (int half = 0; half < 2; ++half) {
          const int sb = 2 * p + half;
          i32x4 av[2];
#pragma unroll
          for (int s = 0; s < 2; ++s)
            av[s] = *reinterpret_cast<const i32x4 *>(&sm.a[ar[s] * kApitch + sb * 32 + 16 * h]);
#pragma unroll
          for (int s = 0; s < 2; ++s) {
            float fa[16], fs[16];
#pragma unroll
            for (int g = 0; g < 4; ++g) {
              const f32x4 d4 = *reinterpret_cast<const f32x4 *>(&sm.da[sb][rbase[s] + 8 * g]);
              const f32x4 s4 = *reinterpret_cast<const f32x4 *>(&sm.sa[sb][rbase[s] + 8 * g]);
              fa[4 * g] = d4.x; fa[4 * g + 1] = d4.y; fa[4 * g + 2] = d4.z; fa[4 * g + 3] = d4.w;
              fs[4 * g] = s4.x; fs[4 * g + 1] = s4.y; fs[4 * g + 2] = s4.z; fs[4 * g + 3] = s4.w;
            }
#pragma unroll
            for (int t = 0; t < 2; ++t) {
              const i32x16 z = {0};
              const i32x16 c = mfma32(av[s], half ? bhi[t] : blo[t], z);
              const float w = fw[t][sb], wmn = fm[t][sb];
#pragma unroll
              for (int i = 0; i < 16; ++i)
                acc[s][t][i] += w * fa[i] * static_cast<float>(c[i]) - wmn * fs[i];
            }
          }
        }
      }
    } else if constexpr (QT == kTypeQ6_K) {
      float dq[2];
      int scv[2][16];
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const uint8_t *row = &sm.w[bn[t] * kWpitch];
        dq[t] = h2f(*reinterpret_cast<const uint16_t *>(row + 208));
        const u32x4 s4 = *reinterpret_cast<const u32x4 *>(row + 192);
        const uint32_t sw[4] = {s4.x, s4.y, s4.z, s4.w};
#pragma unroll
        for (int j = 0; j < 16; ++j)
          scv[t][j] = static_cast<int8_t>((sw[j >> 2] >> (8 * (j & 3))) & 0xFFu);
      }
#pragma unroll
      for (int g = 0; g < 2; ++g) {
#pragma unroll
        for (int sub = 0; sub < 4; ++sub) {
          const int sb = g * 4 + sub;  // Q8_1 block within the super-block
          // 16-value group u (0/1): values 16u..16u+15 of this 32-run; this
          // lane supplies values 16u + 8h .. 16u + 8h + 7.
          int64_t bq[2][2];
#pragma unroll
          for (int t = 0; t < 2; ++t) {
            const uint8_t *row = &sm.w[bn[t] * kWpitch];
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
          }
#pragma unroll
          for (int s = 0; s < 2; ++s) {
            int64_t aq[2];
#pragma unroll
            for (int u = 0; u < 2; ++u)
              aq[u] = *reinterpret_cast<const int64_t *>(&sm.a[ar[s] * kApitch + sb * 32 + 16 * u + 8 * h]);
            float fa[16];
#pragma unroll
            for (int gg = 0; gg < 4; ++gg) {
              const f32x4 d4 = *reinterpret_cast<const f32x4 *>(&sm.da[sb][rbase[s] + 8 * gg]);
              fa[4 * gg] = d4.x; fa[4 * gg + 1] = d4.y; fa[4 * gg + 2] = d4.z; fa[4 * gg + 3] = d4.w;
            }
#pragma unroll
            for (int t = 0; t < 2; ++t) {
              const i32x16 z = {0};
              const i32x16 c0 = mfma16(aq[0], bq[t][0], z);
              const i32x16 c1 = mfma16(aq[1], bq[t][1], z);
              const int s0 = scv[t][g * 8 + 2 * sub], s1 = scv[t][g * 8 + 2 * sub + 1];
              const float dd = dq[t];
#pragma unroll
              for (int i = 0; i < 16; ++i) {
                const int ci = c0[i] * s0 + c1[i] * s1;
                acc[s][t][i] += dd * fa[i] * static_cast<float>(ci);
              }
            }
          }
        }
      }
    } else {
#pragma unroll
      for (int b = 0; b < 8; ++b) {
        i32x4 bw[2];
        float dwv[2];
#pragma unroll
        for (int t = 0; t < 2; ++t) {
          bw[t] = *reinterpret_cast<const i32x4 *>(&sm.w[bn[t] * kWpitch + b * 32 + 16 * h]);
          dwv[t] = sm.dw[b][bn[t]];
        }
#pragma unroll
        for (int s = 0; s < 2; ++s) {
          const i32x4 av = *reinterpret_cast<const i32x4 *>(&sm.a[ar[s] * kApitch + b * 32 + 16 * h]);
          float fa[16];
#pragma unroll
          for (int gg = 0; gg < 4; ++gg) {
            const f32x4 d4 = *reinterpret_cast<const f32x4 *>(&sm.da[b][rbase[s] + 8 * gg]);
            fa[4 * gg] = d4.x; fa[4 * gg + 1] = d4.y; fa[4 * gg + 2] = d4.z; fa[4 * gg + 3] = d4.w;
          }
#pragma unroll
          for (int t = 0; t < 2; ++t) {
            const i32x16 z = {0};
            const i32x16 c = mfma32(av, bw[t], z);
#pragma unroll
            for (int i = 0; i < 16; ++i) acc[s][t][i] += dwv[t] * fa[i] * static_cast<float>(c[i]);
          }
        }
      }
    }
  }

  // Epilogue: lane holds column n and rows rbase + 8g + j.
#pragma unroll
  for (int s = 0; s < 2; ++s)
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const int n = n0 + wn * 64 + 32 * t + l32;
      if (n >= N) continue;
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int m = m0 + wm * 64 + 32 * s + 8 * (i >> 2) + 4 * h + (i & 3);
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

template <int QT>
static hipError_t launch_qt(const uint8_t *W, const uint8_t *A, void *Y, const void *bias, bool f16,
                            int M, int N, int K, int mode, hipStream_t s) {
  const dim3 grid((N + kBN - 1) / kBN, (M + kBM - 1) / kBM);
  const size_t shm = sizeof(Smem);
  // The staged tiles exceed the 64 KiB default; gfx950 has 160 KiB of LDS.
  static bool attr_set[2] = {false, false};
  if (!attr_set[f16]) {
    const void *fn = f16 ? reinterpret_cast<const void *>(&k_gemm_mfma<QT, true>)
                         : reinterpret_cast<const void *>(&k_gemm_mfma<QT, false>);
    const hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize,
                                             static_cast<int>(shm));
    if (e != hipSuccess) return e;
    attr_set[f16] = true;
  }
  if (f16)
    hipLaunchKernelGGL((k_gemm_mfma<QT, true>), grid, dim3(256), shm, s, W, A, Y, bias, M, N, K, mode);
  else
    hipLaunchKernelGGL((k_gemm_mfma<QT, false>), grid, dim3(256), shm, s, W, A, Y, bias, M, N, K, mode);
  return hipGetLastError();
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
