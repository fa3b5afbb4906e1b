// ifx_q8_1.h -- the Q8_1 block quantizer shared by the activation
// quantizer, the fused Q8_1 producers and the fused gate/up GEMV epilogue.
//
// Semantics of the reference quantizer
// (runtime/backends/cuda/native/kernels/fused_dequant_gemv.cuh:597-655), per
// block of 32 values held by 8 lanes (4 each):
//   amax = max|x|; d = amax / 127; inv = amax > 0 ? 127 / amax : 0;
//   q = clamp(rint(x * inv), -128, 127); ds = {f16(d), f16(d * sum(q))}
// in IEEE fp32 with no contraction, so codes and scales are bit-exact with
// the CPU restatement.  The 8 lanes of a block must be active together.
#pragma once

#include "ifx_common.h"

namespace ifx {

#pragma clang fp contract(off)
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

#pragma clang fp contract(on)

}  // namespace ifx
