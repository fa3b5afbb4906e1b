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

// Tiled down-projection weights (weight_map.h:30-36): `data` is the layout
// BuildDownProjMmqLayout wrote, quant_type the GGUF id of the raw weights,
// rows x cols the logical [N][K] shape, tile_cols the rows per tile.
struct MmqWeightInfo {
  const void *data{nullptr};
  int quant_type{-1};
  int rows{0};
  int cols{0};
  int tile_cols{0};
};

// The subset of NativeExecutionPolicy (native_execution_policy.h:11-78)
// that governs this path, with the reference's defaults and environment
// names (FromEnv), except enable_downproj_mmq (below).  The three
// reduction fields are this library's own.
struct NativeExecutionPolicy {
  bool force_cublas{false};                   // INFERFLUX_FORCE_CUBLAS
  bool disable_prepacked_activations{false};  // INFERFLUX_DISABLE_PREPACKED_ACTIVATIONS
  bool disable_q81_activations{false};        // INFERFLUX_DISABLE_Q8_1_ACTIVATIONS
  bool disable_fused_gemv{false};             // INFERFLUX_DISABLE_FUSED_GEMV
  bool enable_experimental_q81_downproj_hot_fixed{false};
  bool enable_experimental_q81_downproj_rowpair_hot_fixed{false};
  bool enable_experimental_q81_grouped_hot_q4k{true};
  bool enable_experimental_q81_grouped_rowpair_w4{true};
  bool enable_experimental_q81_grouped_rowquad_m4{false};
  bool enable_experimental_q81_grouped_mmq3{true};
  // INFERFLUX_ENABLE_DOWNPROJ_MMQ.  The reference defaults it off (its MMQ
  // down projection is an additive migration path); on gfx950 the re-tiled
  // copy is the fastest form of the down projection at every decode M
  // (row-split rows at M <= 2, tiles from M = 3), so it defaults on here.
  bool enable_downproj_mmq{true};
  int downproj_mmq_min_batch_override{-1};    // INFERFLUX_DOWNPROJ_MMQ_MIN_BATCH, 1..64
  bool enable_fused_gate_up_silu{true};       // INFERFLUX_ENABLE_FUSED_GATE_UP_SILU
  // Deterministic K splits (no reference counterpart).  Where a kernel
  // splits K over workgroups, the plain launches add the splits' partial sums
  // with fp32 atomics (as the reference's accumulate kernels), so the last
  // bits vary run to run.
  //  * Gemv* / GemvQ8_1Pair / GemvQ8_1Triple add them in split order
  //    through reduction_workspace (caller-owned device memory, 256-byte
  //    aligned, zeroed once after allocation, ReductionWorkspaceBytes for
  //    the launch) whenever it is given and large enough, so a caller that
  //    provides scratch gets the same bits on every call (launches that need
  //    none take the same deterministic kernels); with
  //    deterministic_reductions set that holds without a workspace too, and
  //    a split launch without a large enough one is not handled (false);
  //    otherwise the launch takes the plain entry and its atomics.
  //  * DownProjMmq* add them in split order through the layout's own
  //    workspace with deterministic_reductions set (fp16 outputs always do);
  //    otherwise with atomics, which are faster there (14B down at M = 32:
  //    about 20 against 25 us).
  // Calls that share a workspace (or a layout) must not overlap.
  bool deterministic_reductions{false};
  void *reduction_workspace{nullptr};
  int64_t reduction_workspace_bytes{0};
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
  // Rows per tile of the down-projection layout: 32, the row count of one
  // v_mfma_i32_32x32x32_i8 operand (the reference's CUDA tile is 8 rows,
  // fused_quant_gemm.h:49).
  static constexpr int kDownProjMmqTileCols = 32;
  // Largest M DownProjMmq handles (the batch kernels on tiles); above it the
  // prefill GEMM on the raw rows (GemvQ8_1) is faster.
  static constexpr int kDownProjMmqMaxM = 32;

  // fused_quant_gemm.h:51-58: grouped gate+up operator labels.
  enum class FfnProjOperator {
    kFallback = 0,
    kQ81Group,
    kQ81GroupHotQ4K,
    kQ81GroupRowPairW4,
    kQ81GroupRowQuadM4,
    kQ81GroupMmq3,
    kPackedGroup,
  };

  // fused_quant_gemm.h:61-70: down-projection operator labels.
  enum class DownProjOperator {
    kFallback = 0,
    kQ81Gemv,
    kQ81GemvHotFixed,
    kQ81GemvRowPairHotFixed,
    kQ81GemvRowPair,
    kQ81GemvRowQuad,
    kPackedGemv,
    kMmq,
  };

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
  // selected_op (fused_quant_gemm.h:272-276) names the reference kernel a
  // selector chose; here every operator runs the kernel ifx_qgemv_grouped
  // routes the geometry to, so it only has to be a valid label.
  static bool GemvQ8_1Pair(const std::array<PackedProjectionSpec, 2> &projections,
                           const void *act_q8_1, int M, int K, hipStream_t stream,
                           const NativeExecutionPolicy *policy = nullptr,
                           FfnProjOperator selected_op = FfnProjOperator::kFallback);
  // fused_quant_gemm.h:285-287: the row-quad candidate, outside selection;
  // the same grouped launch.
  static bool GemvQ8_1PairRowQuadCandidate(const std::array<PackedProjectionSpec, 2> &projections,
                                           const void *act_q8_1, int M, int K,
                                           hipStream_t stream);
  static bool GemvQ8_1Triple(const std::array<PackedProjectionSpec, 3> &projections,
                             const void *act_q8_1, int M, int K, hipStream_t stream,
                             const NativeExecutionPolicy *policy = nullptr);

  // ---- Down projection on the re-tiled copy (fused_quant_gemm.h:213-234) ----
  // output(half) = W . a on a layout from BuildDownProjMmqLayout, N ==
  // weight.rows, K == weight.cols, 1 <= M <= kDownProjMmqMaxM: M <= 2 runs
  // the v_dot4 GEMV on the layout's row-major copy, larger M the batch
  // kernels on its tiles (K splits of fp16 outputs reduced in order through
  // the layout's workspace, so calls on one layout must not overlap).  False
  // (nothing launched) when the policy disables it, the layout does not
  // match or M is out of range.
  static bool DownProjMmq(const MmqWeightInfo &weight, const void *act_q8_1, uint16_t *output,
                          int M, int N, int K, hipStream_t stream,
                          const NativeExecutionPolicy *policy = nullptr);
  // fp32 out, and fp32 `+=` into the residual stream (the decode layer's
  // down projection; no reference counterpart, cf. GemvQ8_1AccumF32).
  static bool DownProjMmqF32(const MmqWeightInfo &weight, const void *act_q8_1, float *output,
                             int M, int N, int K, hipStream_t stream,
                             const NativeExecutionPolicy *policy = nullptr);
  static bool DownProjMmqAccumF32(const MmqWeightInfo &weight, const void *act_q8_1,
                                  float *output, int M, int N, int K, hipStream_t stream,
                                  const NativeExecutionPolicy *policy = nullptr);
  static bool IsDownProjMmqEnabled(const NativeExecutionPolicy *policy = nullptr);
  // Allocates the layout (hipMalloc: tiles + row-major copy, see
  // ifx_mmq_layout_bytes), writes it from the raw rows x cols weights on
  // `stream` and waits for it, as the reference does.  The caller owns it
  // and frees it with DestroyDownProjMmqLayout.
  static bool BuildDownProjMmqLayout(const QuantizedWeightInfo &weight, int rows, int cols,
                                     MmqWeightInfo *layout, hipStream_t stream);
  static void DestroyDownProjMmqLayout(const MmqWeightInfo &layout);
  // Q4_K and Q6_K, as the reference.
  static bool SupportsDownProjMmq(int quant_type);
  // Smallest M at which the tiled path is selected (the policy's override
  // first, else 3: measured on MI355X, tiles win from M = 3, 3B down 2048 x
  // 11008 Q6_K M = 4 8.3 against 12.2 us raw).
  static int GetDownProjMmqThreshold(int quant_type, int m, int n, int k);

  // ---- Operator selection (fused_quant_gemm.h:236-266) ----
  static FfnProjOperator SelectFfnProjOperator(int quant_type0, int quant_type1,
                                               const FusedDispatchGeometry &geometry,
                                               bool allow_q81, bool allow_packed,
                                               const NativeExecutionPolicy *policy = nullptr);
  static const char *FfnProjOperatorName(FfnProjOperator op);
  static const char *FfnProjOperatorMetricName(FfnProjOperator op, int quant_type, int m, int k);
  static DownProjOperator SelectDownProjOperator(int quant_type,
                                                 const FusedDispatchGeometry &geometry,
                                                 bool allow_q81, bool allow_packed,
                                                 bool allow_mmq,
                                                 const NativeExecutionPolicy *policy = nullptr);
  static const char *DownProjOperatorName(DownProjOperator op);
  static const char *DownProjOperatorMetricName(DownProjOperator op, int quant_type, int m,
                                                int k);
  // fused_quant_gemm.h:341-360: the reference's named hot geometries (Q4_K
  // gate+up at K = 2048, N >= 8192, M = 1 / 2; the 2048 x 11008 down
  // projection at M = 1 / 2).  Labels for the selectors; on gfx950 these
  // shapes run the kernels the router picks for them.
  static bool ShouldUseSpecializedQ8_1GroupedFastPath(
      int quant_type, const FusedDispatchGeometry &geometry,
      const NativeExecutionPolicy *policy = nullptr);
  static bool ShouldUseSpecializedQ8_1GroupedRowPairW4Path(
      int quant_type, const FusedDispatchGeometry &geometry,
      const NativeExecutionPolicy *policy = nullptr);
  static bool ShouldUseSpecializedQ8_1DownProjHotPath(
      int quant_type, const FusedDispatchGeometry &geometry,
      const NativeExecutionPolicy *policy = nullptr);
  static bool ShouldUseSpecializedQ8_1DownProjRowPairHotPath(
      int quant_type, const FusedDispatchGeometry &geometry,
      const NativeExecutionPolicy *policy = nullptr);

  // ---- Producers fused into their consumer (no single-call counterpart) ----
  // FusedRmsNormQuantizeQ8_1 followed by GemvQ8_1Pair / GemvQ8_1Triple
  // (transformer_forward.cu:524-559) as one launch: every workgroup forms
  // the Q8_1 activations of RMSNorm(residual) * norm_weight in LDS, bitwise
  // what FusedRmsNormQuantizeQ8_1 writes.  Q4_K, M <= 2 (the geometry
  // ShouldUseFusedPath accepts with includes_rmsnorm); false otherwise, and
  // the caller takes the two calls.
  static bool FusedRmsNormGemvQ8_1Pair(const std::array<PackedProjectionSpec, 2> &projections,
                                       const float *residual, const uint16_t *norm_weight,
                                       int M, int K, float rms_norm_eps, hipStream_t stream,
                                       const NativeExecutionPolicy *policy = nullptr);
  static bool FusedRmsNormGemvQ8_1Triple(const std::array<PackedProjectionSpec, 3> &projections,
                                         const float *residual, const uint16_t *norm_weight,
                                         int M, int K, float rms_norm_eps, hipStream_t stream,
                                         const NativeExecutionPolicy *policy = nullptr);
  // QuantizeRowQ8_1 followed by GemvQ8_1AccumF32 (the O projection into the
  // fp32 residual, transformer_forward.cu:609-726) as one launch.  Q4_K,
  // M <= 2.
  static bool QuantizeGemvQ8_1AccumF32(const QuantizedWeightInfo &weight, const float *input,
                                       float *output, int M, int N, int K, hipStream_t stream,
                                       const NativeExecutionPolicy *policy = nullptr);
  static bool QuantizeGemvQ8_1AccumF32(const QuantizedWeightInfo &weight, const uint16_t *input,
                                       float *output, int M, int N, int K, hipStream_t stream,
                                       const NativeExecutionPolicy *policy = nullptr);
  // FusedRmsNormQuantizeQ8_1 followed by FusedGateUpSiluGemvQ8_1WithEpilogue
  // (transformer_forward.cu:2839-2870) as one launch.  Q4_K, M <= 2,
  // K <= 2048, N % 32 == 0.
  static bool FusedRmsNormGateUpSiluGemvQ8_1WithEpilogue(
      const QuantizedWeightInfo &gate_raw, const QuantizedWeightInfo &up_raw,
      const float *residual, const uint16_t *norm_weight, float rms_norm_eps, uint16_t *output,
      void *act_q8_1_out, int M, int N, int K, hipStream_t stream);

  // Bytes of reduction workspace one launch needs (0: it does not split K);
  // count = number of grouped projections, N[i] their rows.
  static int64_t ReductionWorkspaceBytes(int quant_type, int count, const int *N, bool f16_out,
                                         int M, int K);

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
