// ifx_fused_quant_gemm.h -- C++ host mirror of InferFlux's FusedQuantGemm
// (runtime/backends/cuda/native/fused_quant_gemm.h:47-398) over the gfx950
// C ABI of ifx_qgemm.h.
//
// Same class, method names, argument meaning and error convention as the
// reference: every Gemv* returns true when it enqueued the kernels on
// `stream`, false when it did not handle the call (null pointer, unsupported
// quant type, bad geometry, policy) so the caller takes its fallback.  fp16
// buffers are passed as uint16_t (IEEE binary16 bits), the reference's
// `half`; streams are hipStream_t.  Everything is stream ordered, nothing
// allocates device memory and nothing synchronises the host.
#ifndef IFX_FUSED_QUANT_GEMM_H
#define IFX_FUSED_QUANT_GEMM_H

#include <hip/hip_runtime_api.h>

#include <array>
#include <cstdint>

namespace inferflux {
namespace rocm {

// GGUF tensor type ids (runtime/backends/cuda/native/gguf_util.h:48-63).
enum class TensorType : int { Q8_0 = 8, Q8_1 = 9, Q4_K = 12, Q5_K = 13, Q6_K = 14, Q8_K = 15 };

// Raw quantized weight view (runtime/backends/cuda/native/weight_map.h:17-21).
// Row r of an [N][K] tensor starts at data + r * (K / QK) * block_bytes.
struct QuantizedWeightInfo {
  const void *data{nullptr};
  int quant_type{-1};
  int64_t num_elements{0};
};

// Packed activations (fused_quant_gemm.h:16-19): per-row symmetric int8
// codes [M][K] and one fp32 scale per row (QuantizeRowsSymmetric).
struct PackedActivationInfo {
  const int8_t *data{nullptr};
  const float *row_scales{nullptr};
};

// One output of a grouped launch (fused_quant_gemm.h:22-26); `output` is fp16.
struct PackedProjectionSpec {
  QuantizedWeightInfo weight;
  uint16_t *output{nullptr};
  int output_cols{0};
};

// Shape of a dispatch decision (fused_quant_gemm.h:28-35).
struct FusedDispatchGeometry {
  int M{0};
  int N{0};
  int K{0};
  int grouped_outputs{1};
  bool packed_activation{false};
  bool includes_rmsnorm{false};
};

// The subset of NativeExecutionPolicy (native_execution_policy.h:18, 61-78)
// that governs this path.  FromEnv reads INFERFLUX_DISABLE_FUSED_GEMV.
struct NativeExecutionPolicy {
  bool disable_fused_gemv{false};
  static NativeExecutionPolicy FromEnv();
};

// Which gfx950 kernel family a (quant type, M, N, K) runs on.
enum class KernelFamily : int {
  kNone = 0,
  kGemv = 1,
  kSkinnyMfma = 2,
  kTiledMfma = 3,
  kF16DequantMfma = 4,  // fp16 MFMA with in-kernel dequant (prefill; M >= 33 Q6_K, 96 Q4_K, 128 Q8_0)
  kF16DequantGemv = 5   // fp16 dequant MFMA GEMV (decode batches 17 <= M <= 32)
};

class FusedQuantGemm {
 public:
  // Largest M the quantized path accepts.  The reference stops at 64
  // (kernels/quant_common.cuh:16) and falls back to dequantize + FP16 cuBLAS
  // above it; on gfx950 the int8 MFMA GEMM handles every M, reading 3.6x
  // fewer weight bytes than the FP16 fallback at twice its MFMA rate, so
  // there is no crossover to a fallback.
  static constexpr int kMaxFusedM = 1 << 24;

  // fused_quant_gemm.h:118-119: fp16 [M][K] -> Q8_1 [M][K/32].
  static void QuantizeRowQ8_1(const uint16_t *input, void *output_q8_1, int M, int K,
                              hipStream_t stream);
  // fp32 input variant (the BASELINE contract).
  static void QuantizeRowQ8_1(const float *input, void *output_q8_1, int M, int K,
                              hipStream_t stream);

  // fused_quant_gemm.h:121-129: SiLU(gate) * up quantized to Q8_1 (fp16
  // inputs), and the fp32 variant for fp32 gate/up outputs.
  static void SiluMulQuantizeQ8_1(const uint16_t *gate, const uint16_t *up, void *output_q8_1,
                                  int M, int K, hipStream_t stream);
  static void SiluMulQuantizeQ8_1(const float *gate, const float *up, void *output_q8_1, int M,
                                  int K, hipStream_t stream);
  // fused_quant_gemm.h:131-150: RMSNorm (fp16 norm weights) then Q8_1, for
  // an fp16 or an fp32 residual stream.
  static void FusedRmsNormQuantizeQ8_1(const uint16_t *residual, const uint16_t *norm_weight,
                                       void *output_q8_1, int M, int K, float rms_norm_eps,
                                       hipStream_t stream);
  static void FusedRmsNormQuantizeQ8_1(const float *residual, const uint16_t *norm_weight,
                                       void *output_q8_1, int M, int K, float rms_norm_eps,
                                       hipStream_t stream);

  // fused_quant_gemm.h:171-173: output = W . a, fp16 out.
  static bool GemvQ8_1(const QuantizedWeightInfo &weight, const void *act_q8_1,
                       uint16_t *output, int M, int N, int K, hipStream_t stream,
                       const NativeExecutionPolicy *policy = nullptr);
  // fp32 out (the BASELINE contract; no reference counterpart).
  static bool GemvQ8_1F32(const QuantizedWeightInfo &weight, const void *act_q8_1,
                          float *output, int M, int N, int K, hipStream_t stream,
                          const NativeExecutionPolicy *policy = nullptr);
  // fused_quant_gemm.h:190-193: output(half) += W . a.
  static bool GemvQ8_1Accum(const QuantizedWeightInfo &weight, const void *act_q8_1,
                            uint16_t *output, int M, int N, int K, hipStream_t stream,
                            const NativeExecutionPolicy *policy = nullptr);
  // fused_quant_gemm.h:202-205: output(float) += W . a.
  static bool GemvQ8_1AccumF32(const QuantizedWeightInfo &weight, const void *act_q8_1,
                               float *output, int M, int N, int K, hipStream_t stream,
                               const NativeExecutionPolicy *policy = nullptr);
  // fused_quant_gemm.h:317-328: output = W . a + bias (bias fp16 [N], may be
  // null: then a plain GemvQ8_1).  All three quant types (the reference: Q4_K).
  static bool GemvQ8_1WithBias(const QuantizedWeightInfo &weight, const void *act_q8_1,
                               uint16_t *output, const uint16_t *bias, int M, int N, int K,
                               hipStream_t stream,
                               const NativeExecutionPolicy *policy = nullptr);
  // fused_quant_gemm.h:272-276 / 309-313: sibling projections sharing one
  // Q8_1 activation (gate+up, Q+K+V) in one launch.  N of projection i is
  // projections[i].output_cols.  All must have the same quant type.
  static bool GemvQ8_1Pair(const std::array<PackedProjectionSpec, 2> &projections,
                           const void *act_q8_1, int M, int K, hipStream_t stream,
                           const NativeExecutionPolicy *policy = nullptr);
  static bool GemvQ8_1Triple(const std::array<PackedProjectionSpec, 3> &projections,
                             const void *act_q8_1, int M, int K, hipStream_t stream,
                             const NativeExecutionPolicy *policy = nullptr);

  // fused_quant_gemm.h:281-307: silu(gate . a) * (up . a) in one launch, fp16
  // out; the WithEpilogue variant also writes the Q8_1 blocks of the result
  // (act_q8_1_out, may be null) for the down projection.  N % 32 == 0 and
  // M <= 2, 3 <= M <= 8 for Q4_K / Q6_K with K % 256 == 0, and up to M = 32
  // (Q4_K / Q6_K / Q8_0) where the fp16-dequant GEMV needs no K split (else
  // false: grouped GEMV + SiluMulQuantizeQ8_1, or ifx_qgemv_gate_up_silu_ws
  // with a workspace).
  static bool FusedGateUpSiluGemvQ8_1(const QuantizedWeightInfo &gate_raw,
                                      const QuantizedWeightInfo &up_raw, const void *act_q8_1,
                                      uint16_t *output, int M, int N, int K, hipStream_t stream);
  static bool FusedGateUpSiluGemvQ8_1WithEpilogue(const QuantizedWeightInfo &gate_raw,
                                                  const QuantizedWeightInfo &up_raw,
                                                  const void *act_q8_1, uint16_t *output,
                                                  void *act_q8_1_out, int M, int N, int K,
                                                  hipStream_t stream);

  // fused_quant_gemm.h:72-107: the GEMV on packed (per-row symmetric int8)
  // activations, fp16 out; Q4_K, Q6_K, Q8_0, Q8_K (SupportsPackedActivations).
  // False (nothing launched) for other types, bad geometry or a disabled
  // policy, as the reference.
  static bool GemvPacked(const QuantizedWeightInfo &weight, const PackedActivationInfo &activation,
                         uint16_t *output, int M, int N, int K, hipStream_t stream,
                         const NativeExecutionPolicy *policy = nullptr);
  static bool GemvPackedPair(const std::array<PackedProjectionSpec, 2> &projections,
                             const PackedActivationInfo &activation, int M, int K,
                             hipStream_t stream);
  static bool GemvPackedTriple(const std::array<PackedProjectionSpec, 3> &projections,
                               const PackedActivationInfo &activation, int M, int K,
                               hipStream_t stream);
  // fused_quant_gemm.cu:925-928: the types with a packed-activation kernel.
  static bool SupportsPackedActivations(int quant_type);
  // cuda_kernel::QuantizeRowsSymmetric / SiluMulQuantizeRowsSymmetric
  // (cuda_kernels.cu:309-437), fp16 input: the packed activations.
  static bool QuantizeRowsSymmetric(const uint16_t *input, int8_t *output, float *row_scales,
                                    int rows, int cols, hipStream_t stream);
  static bool SiluMulQuantizeRowsSymmetric(const uint16_t *gate, const uint16_t *up,
                                           int8_t *output, float *row_scales, int rows, int cols,
                                           hipStream_t stream);

  // fused_quant_gemm.h:333: Q4_K, Q6_K, Q8_0 and Q8_K as the reference,
  // and Q5_K, for which the reference has no fused kernel.
  static bool SupportsQ8_1Activations(int quant_type);
  // Largest M of the GEMV-only types Q5_K and Q8_K (the reference's Q8_K
  // dispatch limit, fused_quant_gemm.cu:1740-1747).
  static constexpr int kMaxGemvOnlyM = 64;
  // fused_quant_gemm.h:343-348 and .cu:830-880, re-derived for gfx950.
  static int GetAdaptiveThreshold(int quant_type);
  static int GetGeometryAwareThreshold(int quant_type, const FusedDispatchGeometry &geometry);
  // fused_quant_gemm.h:384-391.
  static bool ShouldUseFusedPath(int quant_type, int M);
  static bool ShouldUseFusedPath(int quant_type, const FusedDispatchGeometry &geometry);
  // The kernel family ifx_qgemv dispatches (quant_type, M, N, K) to.
  static KernelFamily SelectKernel(int quant_type, int M, int N, int K);
  static const char *KernelFamilyName(KernelFamily family);
};

}  // namespace rocm
}  // namespace inferflux

#endif  // IFX_FUSED_QUANT_GEMM_H
