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
#include "ifx_q8_1.h"

namespace ifx {

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

// ---------------------------------------------------------------------------
// Fused producers of Q8_1 activations (the steps before the GEMVs of a
// decode layer), with the quantizer above as their last step.
// ---------------------------------------------------------------------------

// RMSNorm then Q8_1 (fused_dequant_gemv.cuh:736-904): per row,
// rms = 1 / sqrt(sum(x^2) / K + eps), y = (x * rms) * w, quantized per 32.
// One workgroup of 256 threads per row: the sum of squares is reduced with
// DPP within each wave and through LDS across the four waves; then 8 lanes
// per Q8_1 block apply the norm and quantize (for K <= 2048 from registers
// loaded with the norm weight in one round trip, else an L2-resident second
// read of the row).  The reference evaluates rsqrtf (an approximation); here the
// square root and division are correctly rounded.
template <bool F16>
__global__ __launch_bounds__(256) void k_rmsnorm_quantize_q8_1(const void *__restrict__ x,
                                                               const uint16_t *__restrict__ w,
                                                               uint8_t *__restrict__ out, int K,
                                                               float eps) {
  __shared__ float part[4];
  const int64_t row = blockIdx.x;
  uint8_t *orow = out + row * (K >> 5) * kQ8_1Bytes;
  if (K <= 2048) {
    // one round trip to memory: the row and the norm weight are loaded
    // together into registers (the same arithmetic as the two-pass form)
    f32x4 xr[2];
    u32x2 wr[2];
    rmsnorm_row_load<F16, 2>(x, row * K, w, K, threadIdx.x, xr, wr);
    rmsnorm_row_finish<2>(xr, wr, orow, K, eps, part, threadIdx.x);
  } else {
    rmsnorm_quantize_row<F16>(x, row * K, w, orow, K, eps, part, threadIdx.x);
  }
}

// The same for 2048 < K <= 16384 in one round trip: 1024 threads, each
// holding 4 x 4 values of the row and of the norm weight in registers.  The
// sum of squares is formed in the 256-thread kernel's order (the fused
// RMSNorm GEMVs reproduce that kernel's bits): every thread writes its
// 4-value terms to LDS, then thread t < 256 adds the terms of elements
// 4t + 1024j in j order, and the wave / workgroup reductions follow as
// there.  Bit for bit the 256-thread kernel's output.
template <bool F16>
__global__ __launch_bounds__(1024) void k_rmsnorm_quantize_q8_1_wide(const void *__restrict__ x,
                                                                     const uint16_t *__restrict__ w,
                                                                     uint8_t *__restrict__ out,
                                                                     int K, float eps) {
  constexpr int kNit = 4;
  __shared__ float terms[4096];  // element group i / 4
  __shared__ float part[4];
  const int64_t row = blockIdx.x;
  uint8_t *orow = out + row * (K >> 5) * kQ8_1Bytes;
  const int tid = threadIdx.x;
  f32x4 xr[kNit];
  u32x2 wr[kNit];
#pragma unroll
  for (int j = 0; j < kNit; ++j) {
    const int i = 4 * tid + 4096 * j;
    if (i < K) {
      xr[j] = load4<F16>(x, row * K + i);
      wr[j] = ldg<u32x2>(w + i);
    }
  }
#pragma unroll
  for (int j = 0; j < kNit; ++j) {
    const int i = 4 * tid + 4096 * j;
    if (i < K) terms[i >> 2] = xr[j].x * xr[j].x + xr[j].y * xr[j].y + xr[j].z * xr[j].z + xr[j].w * xr[j].w;
  }
  __syncthreads();
  if (tid < 256) {
    float ss = 0.0f;
    for (int i = 4 * tid; i < K; i += 4 * 256) ss += terms[i >> 2];
    ss = wave_sum_to63(ss);
    if ((tid & 63) == 63) part[tid >> 6] = ss;
  }
  __syncthreads();
  const float total = (part[0] + part[1]) + (part[2] + part[3]);
  const float rms = 1.0f / __builtin_sqrtf(total / static_cast<float>(K) + eps);
  const int l = tid & 7;
#pragma unroll
  for (int j = 0; j < kNit; ++j) {
    const int i = 4 * tid + 4096 * j;  // = 32 * block + 4 * l; whole blocks (K % 32 == 0)
    if (i < K) {
      const f32x4 v = xr[j];
      const u32x2 wv = wr[j];
      const float y0 = materialize_f32(v.x * rms) * h2f(wv.x & 0xFFFFu);
      const float y1 = materialize_f32(v.y * rms) * h2f(wv.x >> 16);
      const float y2 = materialize_f32(v.z * rms) * h2f(wv.y & 0xFFFFu);
      const float y3 = materialize_f32(v.w * rms) * h2f(wv.y >> 16);
      quantize4_store(y0, y1, y2, y3, orow + (i >> 5) * kQ8_1Bytes, l);
    }
  }
}

// SiLU(gate) * up then Q8_1 (fused_dequant_gemv.cuh:657-734):
// y = (g / (1 + exp(-g))) * u, 8 lanes per Q8_1 block.
template <bool F16>
__global__ __launch_bounds__(256) void k_silu_mul_quantize_q8_1(const void *__restrict__ g,
                                                                const void *__restrict__ u,
                                                                uint8_t *__restrict__ out,
                                                                int64_t nblocks) {
  const int64_t t = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  const int64_t blk = t >> 3;
  const int l = threadIdx.x & 7;
  if (blk >= nblocks) return;
  const f32x4 gv = load4<F16>(g, blk * 32 + l * 4);
  const f32x4 uv = load4<F16>(u, blk * 32 + l * 4);
  const f32x4 y = silu_mul4(gv, uv);
  quantize4_store(y.x, y.y, y.z, y.w, out + blk * kQ8_1Bytes, l);
}

// ---------------------------------------------------------------------------
// Per-row symmetric int8 activations (the reference's packed-activation
// producers, cuda_kernels.cu:309-437): per row, amax = max |y|,
// scale = amax / 127 (0 for a zero row), inv = 1 / scale (0 likewise),
// q = clamp(rint(y * inv), -127, 127), with y = x (QuantizeRowsSymmetric) or
// y = (g / (1 + exp(-g))) * u (SiluMulQuantizeRowsSymmetric).  Inputs fp32,
// fp16 or bf16 (DT 0 / 1 / 2).  One workgroup of 256 threads per row: amax
// is order-independent, so codes and scale are bit-exact with a CPU
// restatement for y = x (the SiLU form differs where exp differs by an ulp).
// ---------------------------------------------------------------------------
template <int DT>
__device__ __forceinline__ float load_dt(const void *p, int64_t i) {
  if constexpr (DT == 0) return static_cast<const float *>(p)[i];
  else if constexpr (DT == 1) return h2f(static_cast<const uint16_t *>(p)[i]);
  else return __builtin_bit_cast(float, static_cast<uint32_t>(static_cast<const uint16_t *>(p)[i]) << 16);
}

template <int DT, bool SILU>
__device__ __forceinline__ float row_value(const void *a, const void *b, int64_t i) {
  if constexpr (SILU) return silu_mul1(load_dt<DT>(a, i), load_dt<DT>(b, i));
  else return load_dt<DT>(a, i);
}

// Four consecutive values (element i, i % 4 == 0) with one 16- or 8-byte load.
template <int DT>
__device__ __forceinline__ f32x4 load4_dt(const void *p, int64_t i) {
  if constexpr (DT == 0) return ldg<f32x4>(static_cast<const float *>(p) + i);
  const u32x2 v = ldg<u32x2>(static_cast<const uint16_t *>(p) + i);
  if constexpr (DT == 1)
    return f32x4{h2f(v.x & 0xFFFFu), h2f(v.x >> 16), h2f(v.y & 0xFFFFu), h2f(v.y >> 16)};
  else
    return f32x4{__builtin_bit_cast(float, v.x << 16), __builtin_bit_cast(float, v.x & 0xFFFF0000u),
                 __builtin_bit_cast(float, v.y << 16), __builtin_bit_cast(float, v.y & 0xFFFF0000u)};
}

template <int DT, bool SILU>
__device__ __forceinline__ f32x4 row_value4(const void *a, const void *b, int64_t i) {
  if constexpr (SILU) return silu_mul4(load4_dt<DT>(a, i), load4_dt<DT>(b, i));
  else return load4_dt<DT>(a, i);
}

__device__ __forceinline__ int sym_code(float y, float inv) {
  return static_cast<int>(fminf(fmaxf(rintf(y * inv), -127.0f), 127.0f));
}

// V4: K % 4 == 0, four values per thread and load (the same per-element
// arithmetic, so the same codes and scale).
template <int DT, bool SILU, bool V4>
__global__ __launch_bounds__(256) void k_quantize_rows_sym(const void *__restrict__ a,
                                                           const void *__restrict__ b,
                                                           int8_t *__restrict__ codes,
                                                           float *__restrict__ scales, int K) {
  __shared__ float wmax[4];
  const int64_t base = static_cast<int64_t>(blockIdx.x) * K;
  const int tid = threadIdx.x;
  float mx = 0.0f;
  if constexpr (V4) {
    for (int i = 4 * tid; i < K; i += 1024) {
      const f32x4 v = row_value4<DT, SILU>(a, b, base + i);
      mx = fmaxf(fmaxf(mx, fmaxf(fabsf(v.x), fabsf(v.y))), fmaxf(fabsf(v.z), fabsf(v.w)));
    }
  } else {
    for (int i = tid; i < K; i += 256) mx = fmaxf(mx, fabsf(row_value<DT, SILU>(a, b, base + i)));
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
  if ((tid & 63) == 0) wmax[tid >> 6] = mx;
  __syncthreads();
  const float amax = fmaxf(fmaxf(wmax[0], wmax[1]), fmaxf(wmax[2], wmax[3]));
  const float scale = amax > 0.0f ? amax / 127.0f : 0.0f;
  const float inv = scale > 0.0f ? 1.0f / scale : 0.0f;
  if (tid == 0) scales[blockIdx.x] = scale;
  if constexpr (V4) {
    for (int i = 4 * tid; i < K; i += 1024) {
      const f32x4 v = row_value4<DT, SILU>(a, b, base + i);
      const uint32_t w = (static_cast<uint32_t>(sym_code(v.x, inv)) & 0xFFu) |
                         ((static_cast<uint32_t>(sym_code(v.y, inv)) & 0xFFu) << 8) |
                         ((static_cast<uint32_t>(sym_code(v.z, inv)) & 0xFFu) << 16) |
                         (static_cast<uint32_t>(sym_code(v.w, inv)) << 24);
      *reinterpret_cast<uint32_t *>(codes + base + i) = w;
    }
  } else {
    for (int i = tid; i < K; i += 256)
      codes[base + i] = static_cast<int8_t>(sym_code(row_value<DT, SILU>(a, b, base + i), inv));
  }
}

// K % 4 == 0 and K <= 16384: 1024 threads, the row's values (SiLU products
// included) computed once into registers, the maximum over the 16 waves in
// LDS, the codes from the registers: one read of the inputs, one exp per
// element.  Same per-element arithmetic as k_quantize_rows_sym.
template <int DT, bool SILU>
__global__ __launch_bounds__(1024) void k_quantize_rows_sym_reg(const void *__restrict__ a,
                                                                const void *__restrict__ b,
                                                                int8_t *__restrict__ codes,
                                                                float *__restrict__ scales, int K) {
  constexpr int kNit = 4;  // 4 x 4 values per thread
  __shared__ float wmax[16];
  const int64_t base = static_cast<int64_t>(blockIdx.x) * K;
  const int tid = threadIdx.x;
  f32x4 v[kNit];
  float mx = 0.0f;
#pragma unroll
  for (int j = 0; j < kNit; ++j) {
    const int i = 4 * tid + 4096 * j;
    if (i < K) {
      v[j] = row_value4<DT, SILU>(a, b, base + i);
      mx = fmaxf(fmaxf(mx, fmaxf(fabsf(v[j].x), fabsf(v[j].y))), fmaxf(fabsf(v[j].z), fabsf(v[j].w)));
    }
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
  if ((tid & 63) == 0) wmax[tid >> 6] = mx;
  __syncthreads();
  float amax = wmax[0];
#pragma unroll
  for (int w = 1; w < 16; ++w) amax = fmaxf(amax, wmax[w]);
  const float scale = amax > 0.0f ? amax / 127.0f : 0.0f;
  const float inv = scale > 0.0f ? 1.0f / scale : 0.0f;
  if (tid == 0) scales[blockIdx.x] = scale;
#pragma unroll
  for (int j = 0; j < kNit; ++j) {
    const int i = 4 * tid + 4096 * j;
    if (i < K) {
      const uint32_t w = (static_cast<uint32_t>(sym_code(v[j].x, inv)) & 0xFFu) |
                         ((static_cast<uint32_t>(sym_code(v[j].y, inv)) & 0xFFu) << 8) |
                         ((static_cast<uint32_t>(sym_code(v[j].z, inv)) & 0xFFu) << 16) |
                         (static_cast<uint32_t>(sym_code(v[j].w, inv)) << 24);
      *reinterpret_cast<uint32_t *>(codes + base + i) = w;
    }
  }
}

hipError_t launch_quantize_rows_sym(const void *a, const void *b, int dtype, int8_t *codes,
                                    float *scales, int M, int K, hipStream_t stream) {
  if (M == 0) return hipSuccess;
  const dim3 grid(M), block(256);
  // The vector forms load four values (16 bytes fp32, 8 bytes fp16 / bf16)
  // and store four codes per access: they need K % 4 == 0 and bases aligned
  // to those sizes (then every row is); other calls take the scalar form.
  const uintptr_t vin = dtype == 0 ? 16 : 8;
  const bool v4 = K % 4 == 0 && reinterpret_cast<uintptr_t>(a) % vin == 0 &&
                  reinterpret_cast<uintptr_t>(b) % vin == 0 &&
                  reinterpret_cast<uintptr_t>(codes) % 4 == 0;
  if (v4 && K <= 16384) {
    const dim3 rblock(1024);
#define IFX_QRSR(DT)                                                                             \
  do {                                                                                           \
    if (b) IFX_LAUNCH(k_quantize_rows_sym_reg, (DT, true), grid, rblock, 0, stream, a, b, codes, \
                      scales, K);                                                                \
    else IFX_LAUNCH(k_quantize_rows_sym_reg, (DT, false), grid, rblock, 0, stream, a, b, codes,  \
                    scales, K);                                                                  \
  } while (0)
    if (dtype == 0) IFX_QRSR(0);
    else if (dtype == 1) IFX_QRSR(1);
    else IFX_QRSR(2);
#undef IFX_QRSR
    return last_error();
  }
#define IFX_QRS2(DT, V4)                                                                        \
  do {                                                                                          \
    if (b) IFX_LAUNCH(k_quantize_rows_sym, (DT, true, V4), grid, block, 0, stream, a, b, codes, \
                      scales, K);                                                               \
    else IFX_LAUNCH(k_quantize_rows_sym, (DT, false, V4), grid, block, 0, stream, a, b, codes,  \
                    scales, K);                                                                 \
  } while (0)
#define IFX_QRS(DT)                 \
  do {                              \
    if (v4) IFX_QRS2(DT, true);     \
    else IFX_QRS2(DT, false);       \
  } while (0)
  if (dtype == 0) IFX_QRS(0);
  else if (dtype == 1) IFX_QRS(1);
  else IFX_QRS(2);
#undef IFX_QRS
#undef IFX_QRS2
  return last_error();
}

hipError_t launch_rmsnorm_quantize_q8_1(const void *x, bool f16, const uint16_t *w, void *out,
                                        int M, int K, float eps, hipStream_t stream) {
  if (M == 0) return hipSuccess;
  if (K > 2048 && K <= 16384) {
    if (f16)
      IFX_LAUNCH(k_rmsnorm_quantize_q8_1_wide, (true), dim3(M), dim3(1024), 0, stream, x, w,
                 static_cast<uint8_t *>(out), K, eps);
    else
      IFX_LAUNCH(k_rmsnorm_quantize_q8_1_wide, (false), dim3(M), dim3(1024), 0, stream, x, w,
                 static_cast<uint8_t *>(out), K, eps);
    return last_error();
  }
  if (f16)
    IFX_LAUNCH(k_rmsnorm_quantize_q8_1, (true), dim3(M), dim3(256), 0, stream, x, w,
                       static_cast<uint8_t *>(out), K, eps);
  else
    IFX_LAUNCH(k_rmsnorm_quantize_q8_1, (false), dim3(M), dim3(256), 0, stream, x, w,
                       static_cast<uint8_t *>(out), K, eps);
  return last_error();
}

hipError_t launch_silu_mul_quantize_q8_1(const void *g, const void *u, bool f16, void *out,
                                         int64_t M, int64_t K, hipStream_t stream) {
  const int64_t nblocks = M * (K / 32);
  if (nblocks == 0) return hipSuccess;
  const dim3 grid(static_cast<unsigned>((nblocks * 8 + 255) / 256));
  if (f16)
    IFX_LAUNCH(k_silu_mul_quantize_q8_1, (true), grid, dim3(256), 0, stream, g, u,
                       static_cast<uint8_t *>(out), nblocks);
  else
    IFX_LAUNCH(k_silu_mul_quantize_q8_1, (false), grid, dim3(256), 0, stream, g, u,
                       static_cast<uint8_t *>(out), nblocks);
  return last_error();
}

hipError_t launch_quantize_q8_1(const void *x, bool f16, void *out, int64_t M, int64_t K,
                                hipStream_t stream) {
  const int64_t nblocks = M * (K / 32);
  if (nblocks == 0) return hipSuccess;
  const int64_t threads = nblocks * 8;
  const dim3 grid(static_cast<unsigned>((threads + 255) / 256));
  if (f16)
    IFX_LAUNCH0(k_quantize_q8_1_f16, grid, dim3(256), 0, stream,
                       static_cast<const uint16_t *>(x), static_cast<uint8_t *>(out), nblocks);
  else
    IFX_LAUNCH0(k_quantize_q8_1_f32, grid, dim3(256), 0, stream,
                       static_cast<const float *>(x), static_cast<uint8_t *>(out), nblocks);
  return last_error();
}

}  // namespace ifx
