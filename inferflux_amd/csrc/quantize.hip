// quantize.hip -- fp32/fp16 activations -> Q8_1 blocks of 32 on gfx950.
//
// Semantics of the reference quantizer
// (runtime/backends/cuda/native/kernels/fused_dequant_gemv.cuh:597-655), per
// block of 32 values:
//   amax = max|x|; d = amax / 127; inv = amax > 0 ? 127 / amax : 0;
//   q = clamp(rint(x * inv), -128, 127); ds = {f16(d), f16(d * sum(q))}
// evaluated in IEEE fp32 (this file is compiled with -ffp-contract=off and
// HIP's default correctly rounded fp32 division), so codes and scales are
// bit-exact with the CPU restatement.
//
// Mapping: 8 lanes per Q8_1 block, 4 values per lane (one 16-byte load of
// fp32 or 8-byte load of fp16), so a wave64 quantizes 8 blocks and every
// load and store of a wave is contiguous.  amax and sum(q) are reduced
// across the 8 lanes with xor shuffles that stay inside the 8-lane group.
#include "ifx_common.h"

namespace ifx {

__device__ __forceinline__ void quantize4_store(float x0, float x1, float x2, float x3,
                                                uint8_t *blk, int l) {
  float amax = fmaxf(fmaxf(fabsf(x0), fabsf(x1)), fmaxf(fabsf(x2), fabsf(x3)));
  amax = fmaxf(amax, __shfl_xor(amax, 4));
  amax = fmaxf(amax, __shfl_xor(amax, 2));
  amax = fmaxf(amax, __shfl_xor(amax, 1));
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
  sum += __shfl_xor(sum, 4);
  sum += __shfl_xor(sum, 2);
  sum += __shfl_xor(sum, 1);
  const uint32_t packed = (static_cast<uint32_t>(q0) & 0xFFu) |
                          ((static_cast<uint32_t>(q1) & 0xFFu) << 8) |
                          ((static_cast<uint32_t>(q2) & 0xFFu) << 16) |
                          ((static_cast<uint32_t>(q3) & 0xFFu) << 24);
  *reinterpret_cast<uint32_t *>(blk + 4 + 4 * l) = packed;
  if (l == 0) {
    const float s = materialize_f32(d * static_cast<float>(sum));  // fp32 first, then fp16
    const uint32_t ds = f2h_bits(d) | (f2h_bits(s) << 16);
    *reinterpret_cast<uint32_t *>(blk) = ds;
  }
}

// x: [nblocks * 32] fp32, out: [nblocks] Q8_1.  nblocks = M * K / 32.
__global__ __launch_bounds__(256) void k_quantize_q8_1_f32(const float *__restrict__ x,
                                                           uint8_t *__restrict__ out,
                                                           int64_t nblocks) {
  const int64_t t = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  const int64_t blk = t >> 3;
  const int l = threadIdx.x & 7;
  // Lanes exit in whole groups of 8 (blk = t / 8), so every shuffle partner
  // of a live lane is live.
  if (blk >= nblocks) return;
  const f32x4 v = ldg<f32x4>(x + blk * 32 + l * 4);
  quantize4_store(v.x, v.y, v.z, v.w, out + blk * kQ8_1Bytes, l);
}

__global__ __launch_bounds__(256) void k_quantize_q8_1_f16(const uint16_t *__restrict__ x,
                                                           uint8_t *__restrict__ out,
                                                           int64_t nblocks) {
  const int64_t t = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  const int64_t blk = t >> 3;
  const int l = threadIdx.x & 7;
  if (blk >= nblocks) return;
  const u32x2 v = ldg<u32x2>(x + blk * 32 + l * 4);
  quantize4_store(h2f(v.x & 0xFFFFu), h2f(v.x >> 16), h2f(v.y & 0xFFFFu), h2f(v.y >> 16),
                  out + blk * kQ8_1Bytes, l);
}

hipError_t launch_quantize_q8_1(const void *x, bool f16, void *out, int64_t M, int64_t K,
                                hipStream_t stream) {
  const int64_t nblocks = M * (K / 32);
  if (nblocks == 0) return hipSuccess;
  const int64_t threads = nblocks * 8;
  const dim3 grid(static_cast<unsigned>((threads + 255) / 256));
  if (f16)
    hipLaunchKernelGGL(k_quantize_q8_1_f16, grid, dim3(256), 0, stream,
                       static_cast<const uint16_t *>(x), static_cast<uint8_t *>(out), nblocks);
  else
    hipLaunchKernelGGL(k_quantize_q8_1_f32, grid, dim3(256), 0, stream,
                       static_cast<const float *>(x), static_cast<uint8_t *>(out), nblocks);
  return hipGetLastError();
}

}  // namespace ifx
