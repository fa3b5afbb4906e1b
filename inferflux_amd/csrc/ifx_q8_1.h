// ifx_q8_1.h -- the Q8_1 block quantizer shared by the activation
// quantizer, the fused Q8_1 producers and the fused gate/up GEMV epilogue.
//
// Semantics of the reference quantizer
// (runtime/backends/cuda/native/kernels/fused_dequant_gemv.cuh:597-655), per
// block of 32 values held by 8 lanes (4 each):
//   amax = max|x|; d = amax / 127; inv = amax > 0 ? 127 / amax : 0;
//   q = clamp(rint(x * inv), -128, 127); ds = {f16(d), f16(d * sum(q))}
// in IEEE fp32 with no contraction, so codes and scales are bit-exact with
// the CPU restatement.  The 8 lanes of a block must be active together and
// aligned to 8 within the wave (the DPP moves stay inside each 8 lanes).
#pragma once

#include "ifx_common.h"

namespace ifx {

// Stores of a word that other workgroups of the same launch read:
// device-coherent (a relaxed device-scope atomic store), so no cache
// write-back is needed before a grid barrier.
__device__ __forceinline__ void store_dev(uint32_t *p, uint32_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

#pragma clang fp contract(off)
// DEV: write the block with device-coherent stores (store_dev).
template <bool DEV = false>
__device__ __forceinline__ void quantize4_store_to(float x0, float x1, float x2, float x3,
                                                   uint8_t *codes, uint8_t *ds_p, int l) {
  // max and the integer sum over the 8 lanes of the block: DPP moves
  // (VALU, no LDS round trip): swap pairs, swap pairs of pairs, then the
  // mirror within each 8 lanes pairs every lane with one of the other quad.
  // Both reductions are exact, so the order does not matter.
  float amax = fmaxf(fmaxf(fabsf(x0), fabsf(x1)), fmaxf(fabsf(x2), fabsf(x3)));
  amax = fmaxf(amax, dppf<0xB1>(amax));   // quad_perm [1,0,3,2]
  amax = fmaxf(amax, dppf<0x4E>(amax));   // quad_perm [2,3,0,1]
  amax = fmaxf(amax, dppf<0x141>(amax));  // row_half_mirror
  const float d = amax / 127.0f;
  const float inv = (amax > 0.0f) ? 127.0f / amax : 0.0f;
  int q0 = static_cast<int>(__builtin_rintf(x0 * inv));
  int q1 = static_cast<int>(__builtin_rintf(x1 * inv));
  int q2 = static_cast<int>(__builtin_rintf(x2 * inv));
  int q3 = static_cast<int>(__builtin_rintf(x3 * inv));
  q0 = min(127, max(-128, q0));
  q1 = min(127, max(-128, q1));
  q2 = min(127, max(-128, q2));
  q3 = min(127, max(-128, q3));
  int sum = q0 + q1 + q2 + q3;
  sum += static_cast<int>(dpp<0xB1>(0u, static_cast<uint32_t>(sum)));
  sum += static_cast<int>(dpp<0x4E>(0u, static_cast<uint32_t>(sum)));
  sum += static_cast<int>(dpp<0x141>(0u, static_cast<uint32_t>(sum)));
  const uint32_t packed = (static_cast<uint32_t>(q0) & 0xFFu) |
                          ((static_cast<uint32_t>(q1) & 0xFFu) << 8) |
                          ((static_cast<uint32_t>(q2) & 0xFFu) << 16) |
                          ((static_cast<uint32_t>(q3) & 0xFFu) << 24);
  if constexpr (DEV) store_dev(reinterpret_cast<uint32_t *>(codes + 4 * l), packed);
  else *reinterpret_cast<uint32_t *>(codes + 4 * l) = packed;
  if (l == 0) {
    const float s = materialize_f32(d * static_cast<float>(sum));  // fp32 first, then fp16
    const uint32_t ds = f2h_bits(d) | (f2h_bits(s) << 16);
    if constexpr (DEV) store_dev(reinterpret_cast<uint32_t *>(ds_p), ds);
    else *reinterpret_cast<uint32_t *>(ds_p) = ds;
  }
}

// One Q8_1 block at blk (codes at blk + 4, d | s at blk).
template <bool DEV = false>
__device__ __forceinline__ void quantize4_store(float x0, float x1, float x2, float x3,
                                                uint8_t *blk, int l) {
  quantize4_store_to<DEV>(x0, x1, x2, x3, blk + 4, blk, l);
}

// The LDS activation layout of the fused-producer GEMVs (split): per row of
// K values, the codes of block pairs in 80-byte slots (block 2q at 80 q,
// 2q + 1 at 80 q + 32; the 16-byte pad puts the 64-byte reads of
// consecutive lanes on distinct bank groups), then d | s of block b at
// 80 K / 64 + 4 b.  Every field is read with aligned 16- / 8-byte loads.
__host__ __device__ constexpr int split_row_bytes(int K) { return K / 64 * 80 + K / 8; }
__device__ __forceinline__ uint8_t *split_codes(uint8_t *row, int b) {
  return row + (b >> 1) * 80 + (b & 1) * 32;
}
__device__ __forceinline__ uint8_t *split_ds(uint8_t *row, int K, int b) {
  return row + K / 64 * 80 + 4 * b;
}
// Block b of a row in the layout SPLIT selects.
template <bool SPLIT>
__device__ __forceinline__ void quantize4_row_store(float x0, float x1, float x2, float x3,
                                                    uint8_t *row, int K, int b, int l) {
  if constexpr (SPLIT)
    quantize4_store_to(x0, x1, x2, x3, split_codes(row, b), split_ds(row, K, b), l);
  else
    quantize4_store(x0, x1, x2, x3, row + b * kQ8_1Bytes, l);
}

// fp32 or fp16 (IEEE binary16 bits) activations, four at element i.
template <bool F16>
__device__ __forceinline__ f32x4 load4(const void *p, int64_t i) {
  if constexpr (F16) {
    const u32x2 v = ldg<u32x2>(static_cast<const uint16_t *>(p) + i);
    return f32x4{h2f(v.x & 0xFFFFu), h2f(v.x >> 16), h2f(v.y & 0xFFFFu), h2f(v.y >> 16)};
  } else {
    return ldg<f32x4>(static_cast<const float *>(p) + i);
  }
}

// RMSNorm then Q8_1 of one row (fused_dequant_gemv.cuh:736-904) by a
// workgroup of exactly 256 threads: rms = 1 / sqrt(sum(x^2) / K + eps),
// y = (x * rms) * w, quantized per 32 values into orow (global or LDS).
// The sum of squares is reduced with DPP within each wave and through
// part[0..3] (LDS) across the four waves; then 8 lanes per Q8_1 block apply
// the norm and quantize (a second, cache-resident read of the row, which
// keeps the register count of the GEMV that fuses this low).  Every caller
// (the standalone producer and that GEMV) runs this same code, so their
// codes are identical.  The square root and division are correctly
// rounded (the reference evaluates rsqrtf).
template <bool F16, bool SPLIT = false>
__device__ __forceinline__ void rmsnorm_quantize_row(const void *x, int64_t base,
                                                     const uint16_t *w, uint8_t *orow, int K,
                                                     float eps, float *part, int tid) {
  float ss = 0.0f;
  for (int i = 4 * tid; i < K; i += 4 * 256) {
    const f32x4 v = load4<F16>(x, base + i);
    ss += v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
  }
  ss = wave_sum_to63(ss);
  if ((tid & 63) == 63) part[tid >> 6] = ss;
  __syncthreads();
  const float total = (part[0] + part[1]) + (part[2] + part[3]);
  const float rms = 1.0f / __builtin_sqrtf(total / static_cast<float>(K) + eps);
  const int nblk = K >> 5;
  // whole 8-lane groups per block: every shuffle partner is live
  for (int b = tid >> 3; b < nblk; b += 32) {
    const int l = tid & 7;
    const int i = b * 32 + l * 4;
    const f32x4 v = load4<F16>(x, base + i);
    const u32x2 wv = ldg<u32x2>(w + i);
    const float y0 = materialize_f32(v.x * rms) * h2f(wv.x & 0xFFFFu);
    const float y1 = materialize_f32(v.y * rms) * h2f(wv.x >> 16);
    const float y2 = materialize_f32(v.z * rms) * h2f(wv.y & 0xFFFFu);
    const float y3 = materialize_f32(v.w * rms) * h2f(wv.y >> 16);
    quantize4_row_store<SPLIT>(y0, y1, y2, y3, orow, K, b, l);
  }
}

// The same row in two phases for a kernel that must issue other loads in
// between (a wave's loads complete in issue order, so data loaded after a
// long weight prefetch waits for all of it): rmsnorm_row_load reads the
// thread's elements 4t + 1024j (j < NIT) of x and of the norm weight into
// registers, rmsnorm_row_finish computes exactly what rmsnorm_quantize_row
// computes from them.  Requires K <= 1024 * NIT.
// DEV: x is fp32 written earlier in the same launch by other workgroups:
// device-coherent loads (relaxed device-scope atomic loads).
template <bool F16, int NIT, bool DEV = false>
__device__ __forceinline__ void rmsnorm_row_load(const void *x, int64_t base, const uint16_t *w,
                                                 int K, int tid, f32x4 (&xr)[NIT],
                                                 u32x2 (&wr)[NIT]) {
  static_assert(!(DEV && F16), "device-coherent loads of fp32 rows only");
#pragma unroll
  for (int j = 0; j < NIT; ++j) {
    const int i = 4 * tid + 1024 * j;
    if (i < K) {
      if constexpr (DEV) {
        const float *xf = static_cast<const float *>(x) + base + i;
#pragma unroll
        for (int e = 0; e < 4; ++e)
          xr[j][e] = __hip_atomic_load(xf + e, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      } else {
        xr[j] = load4<F16>(x, base + i);
      }
      if (w) wr[j] = ldg<u32x2>(w + i);  // w == nullptr: plain quantize, no norm weight
    }
  }
}

// rmsnorm_row_load with no branch around the loads, for kernels that issue
// their weight loads right after it: a load under a branch makes the
// compiler wait for every outstanding load (the weights included) at the
// branch's end, before the producer's arithmetic.  Elements past K re-read
// element K - 4 (their values are never used); thread t may be any thread
// id (its low 8 bits select the elements).  HAS_W: load the norm weight.
template <bool F16, int NIT, bool HAS_W>
__device__ __forceinline__ void rmsnorm_row_load_nb(const void *x, int64_t base,
                                                    const uint16_t *w, int K, int tid,
                                                    f32x4 (&xr)[NIT], u32x2 (&wr)[NIT]) {
#pragma unroll
  for (int j = 0; j < NIT; ++j) {
    const int i = min(4 * (tid & 255) + 1024 * j, K - 4);
    xr[j] = load4<F16>(x, base + i);
    if constexpr (HAS_W) wr[j] = ldg<u32x2>(w + i);
  }
}

// rmsnorm_row_finish in two phases around a barrier that the caller
// executes (a workgroup larger than the 256 producer threads runs the
// barrier on every wave): rmsnorm_row_partial writes the four waves' sums of
// squares to part[0..3], rmsnorm_row_apply reads them after the barrier.
template <int NIT>
__device__ __forceinline__ void rmsnorm_row_partial(const f32x4 (&xr)[NIT], int K, float *part,
                                                    int tid) {
  float ss = 0.0f;
#pragma unroll
  for (int j = 0; j < NIT; ++j)
    if (4 * tid + 1024 * j < K)
      ss += xr[j].x * xr[j].x + xr[j].y * xr[j].y + xr[j].z * xr[j].z + xr[j].w * xr[j].w;
  ss = wave_sum_to63(ss);
  if ((tid & 63) == 63) part[tid >> 6] = ss;
}

template <int NIT, bool SPLIT = false>
__device__ __forceinline__ void rmsnorm_row_apply(const f32x4 (&xr)[NIT], const u32x2 (&wr)[NIT],
                                                  uint8_t *orow, int K, float eps,
                                                  const float *part, int tid) {
  const float total = (part[0] + part[1]) + (part[2] + part[3]);
  const float rms = 1.0f / __builtin_sqrtf(total / static_cast<float>(K) + eps);
  const int l = tid & 7;
#pragma unroll
  for (int j = 0; j < NIT; ++j) {
    const int i = 4 * tid + 1024 * j;  // = 32 * block + 4 * l
    if (i < K) {
      const f32x4 v = xr[j];
      const u32x2 wv = wr[j];
      const float y0 = materialize_f32(v.x * rms) * h2f(wv.x & 0xFFFFu);
      const float y1 = materialize_f32(v.y * rms) * h2f(wv.x >> 16);
      const float y2 = materialize_f32(v.z * rms) * h2f(wv.y & 0xFFFFu);
      const float y3 = materialize_f32(v.w * rms) * h2f(wv.y >> 16);
      quantize4_row_store<SPLIT>(y0, y1, y2, y3, orow, K, i >> 5, l);
    }
  }
}

// 256 threads exactly.
template <int NIT, bool SPLIT = false>
__device__ __forceinline__ void rmsnorm_row_finish(const f32x4 (&xr)[NIT], const u32x2 (&wr)[NIT],
                                                   uint8_t *orow, int K, float eps, float *part,
                                                   int tid) {
  rmsnorm_row_partial<NIT>(xr, K, part, tid);
  __syncthreads();
  rmsnorm_row_apply<NIT, SPLIT>(xr, wr, orow, K, eps, part, tid);
}

// SiLU(g) * u (the standalone producer's arithmetic), of one and of four values.
__device__ __forceinline__ float silu_mul1(float g, float u) {
  return materialize_f32(g / (1.0f + expf(-g))) * u;
}
__device__ __forceinline__ f32x4 silu_mul4(f32x4 g, f32x4 u) {
  f32x4 h;
#pragma unroll
  for (int i = 0; i < 4; ++i) h[i] = silu_mul1(g[i], u[i]);
  return h;
}

// Plain Q8_1 of one row (no norm) in the same element-to-thread mapping:
// thread t quantizes elements 4t + 1024j as one of the 8 lanes of their
// block, which is exactly what the standalone quantizer computes per block.
template <int NIT, bool SPLIT = false>
__device__ __forceinline__ void quantize_row_finish(const f32x4 (&xr)[NIT], uint8_t *orow, int K,
                                                    int tid) {
  const int l = tid & 7;
#pragma unroll
  for (int j = 0; j < NIT; ++j) {
    const int i = 4 * tid + 1024 * j;
    if (i < K) quantize4_row_store<SPLIT>(xr[j].x, xr[j].y, xr[j].z, xr[j].w, orow, K, i >> 5, l);
  }
}

template <bool F16, bool SPLIT = false>
__device__ __forceinline__ void quantize_row(const void *x, int64_t base, uint8_t *orow, int K,
                                             int tid) {
  const int l = tid & 7;
  for (int i = 4 * tid; i < K; i += 1024) {
    const f32x4 v = load4<F16>(x, base + i);
    quantize4_row_store<SPLIT>(v.x, v.y, v.z, v.w, orow, K, i >> 5, l);
  }
}

#pragma clang fp contract(on)

}  // namespace ifx
