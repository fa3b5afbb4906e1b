// ifx_native_dispatch.h -- C++ mirror of InferFlux's native dispatch
// registry and policy helpers (runtime/backends/cuda/native/
// native_dispatch_registry.h:1-96, native_dispatch_policy.h:1-47): the rule
// tables behind FusedQuantGemm::SelectFfnProjOperator /
// SelectDownProjOperator and the caller-side wrappers that apply the
// execution policy before selecting.
//
// Same names, enumerators, bucket boundaries, rule order and policy gates
// as the reference, so a forward pass written against it selects the same
// operator label for the same inputs; the thresholds the rules consult
// (ShouldUseFusedPath, GetDownProjMmqThreshold) are this library's, measured
// on MI355X.
#ifndef IFX_NATIVE_DISPATCH_H
#define IFX_NATIVE_DISPATCH_H

#include <string>
#include <string_view>

#include "ifx_fused_quant_gemm.h"

namespace inferflux {
namespace rocm {

enum class InferfluxCudaDispatchPhase { kUnknown = 0, kDecode, kPrefill };

enum class InferfluxCudaDispatchBucket { k1 = 0, k2, k3_4, k5_8, k9_16, k17Plus };

const char *InferfluxCudaDispatchPhaseName(InferfluxCudaDispatchPhase phase);
InferfluxCudaDispatchPhase ParseInferfluxCudaDispatchPhase(std::string_view phase);

InferfluxCudaDispatchBucket BucketBatchRows(int rows);
InferfluxCudaDispatchBucket BucketExtent(int extent);
const char *InferfluxCudaDispatchBucketName(InferfluxCudaDispatchBucket bucket);

struct InferfluxCudaFfnDispatchProfile {
  InferfluxCudaDispatchPhase phase{InferfluxCudaDispatchPhase::kUnknown};
  int quant_type0{0};
  int quant_type1{0};
  FusedDispatchGeometry geometry{};
  bool same_quant{false};
  bool q81_ready{false};
  bool packed_ready{false};
  InferfluxCudaDispatchBucket m_bucket{InferfluxCudaDispatchBucket::k1};
  InferfluxCudaDispatchBucket n_bucket{InferfluxCudaDispatchBucket::k1};
  InferfluxCudaDispatchBucket k_bucket{InferfluxCudaDispatchBucket::k1};
};

struct InferfluxCudaFfnDispatchDecision {
  FusedQuantGemm::FfnProjOperator op{FusedQuantGemm::FfnProjOperator::kFallback};
  const char *reason{nullptr};
};

struct InferfluxCudaDownProjDispatchProfile {
  InferfluxCudaDispatchPhase phase{InferfluxCudaDispatchPhase::kUnknown};
  int quant_type{0};
  FusedDispatchGeometry geometry{};
  bool q81_ready{false};
  bool packed_ready{false};
  bool mmq_ready{false};
  InferfluxCudaDispatchBucket m_bucket{InferfluxCudaDispatchBucket::k1};
  InferfluxCudaDispatchBucket n_bucket{InferfluxCudaDispatchBucket::k1};
  InferfluxCudaDispatchBucket k_bucket{InferfluxCudaDispatchBucket::k1};
};

struct InferfluxCudaDownProjDispatchDecision {
  FusedQuantGemm::DownProjOperator op{FusedQuantGemm::DownProjOperator::kFallback};
  const char *reason{nullptr};
};

InferfluxCudaFfnDispatchProfile BuildInferfluxCudaFfnDispatchProfile(
    InferfluxCudaDispatchPhase phase, int quant_type0, int quant_type1,
    const FusedDispatchGeometry &geometry, bool q81_ready, bool packed_ready);
InferfluxCudaFfnDispatchDecision SelectInferfluxCudaFfnDispatchDecision(
    const InferfluxCudaFfnDispatchProfile &profile, const NativeExecutionPolicy &policy);
std::string DescribeInferfluxCudaFfnDispatchDecision(
    const InferfluxCudaFfnDispatchProfile &profile, std::string_view reason);

InferfluxCudaDownProjDispatchProfile BuildInferfluxCudaDownProjDispatchProfile(
    InferfluxCudaDispatchPhase phase, int quant_type, const FusedDispatchGeometry &geometry,
    bool q81_ready, bool packed_ready, bool mmq_ready);
InferfluxCudaDownProjDispatchDecision SelectInferfluxCudaDownProjDispatchDecision(
    const InferfluxCudaDownProjDispatchProfile &profile, const NativeExecutionPolicy &policy);
std::string DescribeInferfluxCudaDownProjDispatchDecision(
    const InferfluxCudaDownProjDispatchProfile &profile, std::string_view reason);

// native_dispatch_policy.h:13-42.
const NativeExecutionPolicy &ResolveInferfluxCudaExecutionPolicy(
    const NativeExecutionPolicy *policy);
std::string ProjectionQuantLabel(const QuantizedWeightInfo &weight);
std::string ProjectionGroupQuantLabel(const QuantizedWeightInfo &first,
                                      const QuantizedWeightInfo &second);
bool ForceCublasRequested(const NativeExecutionPolicy &policy);
bool PackedActivationsDisabled(const NativeExecutionPolicy &policy);
bool Q81ActivationsDisabled(const NativeExecutionPolicy &policy);
bool ProjectionHasGraphSafeKernel(const QuantizedWeightInfo &raw,
                                  const FusedDispatchGeometry &geometry,
                                  bool allow_fused_quantized_matmul,
                                  const NativeExecutionPolicy &policy);
FusedQuantGemm::DownProjOperator SelectInferfluxCudaDownProjOperator(
    const QuantizedWeightInfo &raw, const MmqWeightInfo &mmq_weight,
    InferfluxCudaDispatchPhase phase, const FusedDispatchGeometry &geometry,
    bool allow_fused_quantized_matmul, const NativeExecutionPolicy &policy);
FusedQuantGemm::FfnProjOperator SelectInferfluxCudaFfnProjOperator(
    const QuantizedWeightInfo &gate_raw, const QuantizedWeightInfo &up_raw,
    InferfluxCudaDispatchPhase phase, const FusedDispatchGeometry &geometry,
    bool allow_fused_quantized_matmul, const NativeExecutionPolicy &policy);

}  // namespace rocm
}  // namespace inferflux

#endif  // IFX_NATIVE_DISPATCH_H
