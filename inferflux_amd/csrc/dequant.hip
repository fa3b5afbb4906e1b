// dequant.hip -- whole-tensor dequantization of raw GGUF blocks on gfx950.
//
// Replaces the reference's dequantize_{q4_k,q5_k,q6_k,q8_0,q8_k} kernels
// (runtime/backends/cuda/native/kernels/dequantization.cu:14-230) and uses
// the element formulas of kernels/quant_common.cuh:100-199:
//   Q4_K  w = d*sc*q - dmin*m      Q6_K  w = d*scale*(q-32)     Q8_0  w = d*q
//   Q5_K  as Q4_K with q = nibble + 16*(bit sb of qh[e])        Q8_K  w = d*q (fp32 d)
// evaluated left to right in IEEE fp32 (this file is compiled with
// -ffp-contract=off), so the values are bit-exact with the CPU restatement.
// The output is fp32, or fp16 (round to nearest even) as the reference
// emits.  It serves verification and callers that want a dense copy; the
// GEMV/GEMM kernels never materialise W.
//
// Mapping: one lane per 32-element run (a Q4_K/Q5_K sub-block, a Q6_K
// (group, sub) run, a Q8_0 block, a Q8_K 32-value slice); each lane writes
// 32 contiguous outputs.
#include "ifx_common.h"

namespace ifx {

// 6-bit scale and min of sub-block sb (quant_common.cuh:83-94).
__device__ __forceinline__ void scale_min_k4(const uint8_t *s, int sb, int &sc, int &m) {
  if (sb < 4) {
    sc = s[sb] & 63;
    m = s[sb + 4] & 63;
  } else {
    sc = (s[sb + 4] & 0xF) | ((s[sb - 4] >> 6) << 4);
    m = (s[sb + 4] >> 4) | ((s[sb] >> 6) << 4);
  }
}

template <int QT, bool F16>
__global__ __launch_bounds__(256) void k_dequant(const uint8_t *__restrict__ W,
                                                 void *__restrict__ out, int64_t nruns) {
  const int64_t t = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (t >= nruns) return;
  float w[32];
  if constexpr (QT == kTypeQ4_K) {
    const int64_t blk = t >> 3;
    const int sb = static_cast<int>(t & 7);
    const uint8_t *b = W + blk * kQ4KBytes;
    const float d = h2f(ldg<uint16_t>(b));
    const float dmin = h2f(ldg<uint16_t>(b + 2));
    int sc, m;
    scale_min_k4(b + 4, sb, sc, m);
    const uint8_t *qs = b + 16 + (sb >> 1) * 32;
    const int shift = (sb & 1) * 4;
#pragma unroll
    for (int e = 0; e < 32; ++e) {
      const int q = (qs[e] >> shift) & 0xF;
      w[e] = d * static_cast<float>(sc) * static_cast<float>(q) - dmin * static_cast<float>(m);
    }
  } else if constexpr (QT == kTypeQ5_K) {
    const int64_t blk = t >> 3;
    const int sb = static_cast<int>(t & 7);
    const uint8_t *b = W + blk * kQ5KBytes;
    const float d = h2f(ldg<uint16_t>(b));
    const float dmin = h2f(ldg<uint16_t>(b + 2));
    int sc, m;
    scale_min_k4(b + 4, sb, sc, m);
    const uint8_t *qh = b + 16;
    const uint8_t *qs = b + 48 + (sb >> 1) * 32;
    const int shift = (sb & 1) * 4;
#pragma unroll
    for (int e = 0; e < 32; ++e) {
      const int q = ((qs[e] >> shift) & 0xF) | (((qh[e] >> sb) & 1) << 4);
      w[e] = d * static_cast<float>(sc) * static_cast<float>(q) - dmin * static_cast<float>(m);
    }
  } else if constexpr (QT == kTypeQ8_K) {
    const int64_t blk = t >> 3;
    const uint8_t *b = W + blk * kQ8KBytes;
    const float d = ldg<float>(b);
    const int8_t *qs = reinterpret_cast<const int8_t *>(b + 4) + (t & 7) * 32;
#pragma unroll
    for (int e = 0; e < 32; ++e) w[e] = d * static_cast<float>(qs[e]);
  } else if constexpr (QT == kTypeQ6_K) {
    const int64_t blk = t >> 3;
    const int run = static_cast<int>(t & 7);
    const int g = run >> 2, sub = run & 3;
    const uint8_t *b = W + blk * kQ6KBytes;
    const float d = h2f(ldg<uint16_t>(b + 208));
    const uint8_t *ql = b + g * 64 + (sub & 1) * 32;
    const uint8_t *qh = b + 128 + g * 32;
    const int8_t *sc = reinterpret_cast<const int8_t *>(b + 192) + g * 8 + sub * 2;
    const int lshift = (sub >= 2) ? 4 : 0;
#pragma unroll
    for (int e = 0; e < 32; ++e) {
      const int q = (((ql[e] >> lshift) & 0xF) | (((qh[e] >> (2 * sub)) & 3) << 4)) - 32;
      w[e] = d * static_cast<float>(sc[e >> 4]) * static_cast<float>(q);
    }
  } else {
    const uint8_t *b = W + t * kQ8_0Bytes;
    const float d = h2f(ldg<uint16_t>(b));
    const int8_t *qs = reinterpret_cast<const int8_t *>(b + 2);
#pragma unroll
    for (int e = 0; e < 32; ++e) w[e] = d * static_cast<float>(qs[e]);
  }
  if constexpr (F16) {
    uint32_t *o = reinterpret_cast<uint32_t *>(static_cast<uint16_t *>(out) + t * 32);
#pragma unroll
    for (int e = 0; e < 32; e += 2)  // fp32 value first, then fp16 (no fused multiply-convert)
      o[e >> 1] = f2h_bits(materialize_f32(w[e])) | (f2h_bits(materialize_f32(w[e + 1])) << 16);
  } else {
    f32x4 *o = reinterpret_cast<f32x4 *>(static_cast<float *>(out) + t * 32);
#pragma unroll
    for (int e = 0; e < 32; e += 4) o[e >> 2] = f32x4{w[e], w[e + 1], w[e + 2], w[e + 3]};
  }
}

template <int QT>
static void launch_dq(const uint8_t *W, void *out, bool f16, int64_t nruns, hipStream_t s) {
  const dim3 grid(static_cast<unsigned>((nruns + 255) / 256));
  if (f16)
    hipLaunchKernelGGL((k_dequant<QT, true>), grid, dim3(256), 0, s, W, out, nruns);
  else
    hipLaunchKernelGGL((k_dequant<QT, false>), grid, dim3(256), 0, s, W, out, nruns);
}

// n_elems must be a multiple of the block size of qtype (checked by caller).
hipError_t launch_dequantize(int qtype, const void *W, void *out, bool f16, int64_t n_elems,
                             hipStream_t stream) {
  const int64_t nruns = n_elems / 32;
  if (nruns == 0) return hipSuccess;
  const uint8_t *w = static_cast<const uint8_t *>(W);
  switch (qtype) {
  case kTypeQ4_K: launch_dq<kTypeQ4_K>(w, out, f16, nruns, stream); break;
  case kTypeQ6_K: launch_dq<kTypeQ6_K>(w, out, f16, nruns, stream); break;
  case kTypeQ8_0: launch_dq<kTypeQ8_0>(w, out, f16, nruns, stream); break;
  case kTypeQ5_K: launch_dq<kTypeQ5_K>(w, out, f16, nruns, stream); break;
  case kTypeQ8_K: launch_dq<kTypeQ8_K>(w, out, f16, nruns, stream); break;
  default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace ifx
