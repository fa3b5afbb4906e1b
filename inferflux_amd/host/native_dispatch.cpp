// native_dispatch.cpp -- the operator-selection rules of InferFlux's native
// backend (native_dispatch_registry.cpp:1-373, native_dispatch_policy.cpp:
// 1-135, and FusedQuantGemm::Select* / *OperatorName / ShouldUseSpecialized*
// of fused_quant_gemm.cu:359-389, 945-1128) over this library's thresholds.
//
// The rules are an ordered list; the first whose readiness requirements hold
// and whose predicate matches names the operator.  Order, predicates, policy
// gates and names are the reference's, so callers pick the same labels;
// readiness comes from this library's ShouldUseFusedPath and
// GetDownProjMmqThreshold, and on gfx950 every Q8_1 label runs the kernel
// the C ABI routes the geometry to.
#include "../../include/ifx_native_dispatch.h"

#include <array>

#include "../../include/ifx_gguf.h"

namespace inferflux {
namespace rocm {

namespace {

using FfnOp = FusedQuantGemm::FfnProjOperator;
using DownOp = FusedQuantGemm::DownProjOperator;
using Ffn = InferfluxCudaFfnDispatchProfile;
using Down = InferfluxCudaDownProjDispatchProfile;
using Policy = NativeExecutionPolicy;

constexpr int kQ4K = static_cast<int>(TensorType::Q4_K);
constexpr int kQ6K = static_cast<int>(TensorType::Q6_K);

// The reference's named hot geometries (fused_quant_gemm.cu:289-291).
constexpr int kGroupedHotK = 2048;
constexpr int kDownHotN = 2048;
constexpr int kDownHotK = 11008;

bool IsDecode(const Ffn &p) { return p.phase == InferfluxCudaDispatchPhase::kDecode; }
bool Q4KPairOfTwo(const Ffn &p) {
  return p.same_quant && p.quant_type0 == kQ4K && p.geometry.grouped_outputs == 2;
}

struct FfnRule {
  FfnOp op;
  bool needs_q81;
  bool needs_packed;
  bool (*match)(const Ffn &, const Policy &);
  const char *reason;
};

struct DownRule {
  DownOp op;
  bool needs_q81;
  bool needs_packed;
  bool needs_mmq;
  bool (*match)(const Down &, const Policy &);
  const char *reason;
};

// native_dispatch_registry.cpp:31-131.
const std::array<FfnRule, 8> &FfnRules() {
  static const std::array<FfnRule, 8> rules = {{
      {FfnOp::kQ81GroupHotQ4K, true, false,
       [](const Ffn &p, const Policy &pol) {
         return IsDecode(p) && p.same_quant &&
                FusedQuantGemm::ShouldUseSpecializedQ8_1GroupedFastPath(p.quant_type0, p.geometry,
                                                                        &pol);
       },
       "decode_q81_hot_q4k"},
      {FfnOp::kQ81GroupRowPairW4, true, false,
       [](const Ffn &p, const Policy &pol) {
         return IsDecode(p) && pol.enable_experimental_q81_grouped_rowpair_w4 && Q4KPairOfTwo(p) &&
                p.m_bucket == InferfluxCudaDispatchBucket::k2 && p.geometry.N >= 8192 &&
                p.geometry.K == kGroupedHotK;
       },
       "decode_q81_rowpair_w4"},
      {FfnOp::kQ81GroupRowQuadM4, true, false,
       [](const Ffn &p, const Policy &pol) {
         return IsDecode(p) && pol.enable_experimental_q81_grouped_rowquad_m4 && Q4KPairOfTwo(p) &&
                p.geometry.M == 4 && p.geometry.N >= 8192 && p.geometry.K == kGroupedHotK;
       },
       "decode_q81_rowquad_m4"},
      {FfnOp::kQ81GroupMmq3, true, false,
       [](const Ffn &p, const Policy &pol) {
         return IsDecode(p) && pol.enable_experimental_q81_grouped_mmq3 && Q4KPairOfTwo(p) &&
                p.geometry.M >= 3;
       },
       "decode_q81_mmq3"},
      {FfnOp::kQ81Group, true, false,
       [](const Ffn &p, const Policy &) { return IsDecode(p) && p.geometry.grouped_outputs == 2; },
       "decode_q81_generic"},
      {FfnOp::kQ81Group, true, false,
       [](const Ffn &p, const Policy &) {
         return p.phase == InferfluxCudaDispatchPhase::kPrefill && p.geometry.grouped_outputs == 2;
       },
       "prefill_q81_generic"},
      {FfnOp::kQ81Group, true, false,
       [](const Ffn &p, const Policy &) {
         return p.phase == InferfluxCudaDispatchPhase::kUnknown && p.geometry.grouped_outputs == 2;
       },
       "q81_generic"},
      {FfnOp::kPackedGroup, false, true,
       [](const Ffn &p, const Policy &) { return p.geometry.grouped_outputs == 2; },
       "packed_group"},
  }};
  return rules;
}

bool Q4KOrQ6K(int t) { return t == kQ4K || t == kQ6K; }

// native_dispatch_registry.cpp:133-206.
const std::array<DownRule, 7> &DownRules() {
  static const std::array<DownRule, 7> rules = {{
      {DownOp::kMmq, false, false, true, [](const Down &p, const Policy &) { return p.mmq_ready; },
       "mmq"},
      {DownOp::kQ81GemvHotFixed, true, false, false,
       [](const Down &p, const Policy &pol) {
         return FusedQuantGemm::ShouldUseSpecializedQ8_1DownProjHotPath(p.quant_type, p.geometry,
                                                                        &pol);
       },
       "q81_hot_fixed"},
      {DownOp::kQ81GemvRowPairHotFixed, true, false, false,
       [](const Down &p, const Policy &pol) {
         return FusedQuantGemm::ShouldUseSpecializedQ8_1DownProjRowPairHotPath(p.quant_type,
                                                                               p.geometry, &pol);
       },
       "q81_rowpair_hot_fixed"},
      {DownOp::kQ81GemvRowQuad, true, false, false,
       [](const Down &p, const Policy &) { return Q4KOrQ6K(p.quant_type) && p.geometry.M >= 4; },
       "q81_rowquad"},
      {DownOp::kQ81GemvRowPair, true, false, false,
       [](const Down &p, const Policy &) { return Q4KOrQ6K(p.quant_type) && p.geometry.M > 1; },
       "q81_rowpair"},
      {DownOp::kQ81Gemv, true, false, false, [](const Down &, const Policy &) { return true; },
       "q81_generic"},
      {DownOp::kPackedGemv, false, true, false, [](const Down &, const Policy &) { return true; },
       "packed_gemv"},
  }};
  return rules;
}

const char *Flag(bool b) { return b ? "true" : "false"; }

std::string TypeLabel(int t) {
  const char *n = ifx_gguf_type_name(t);
  return n ? n : "unknown";
}

}  // namespace

const char *InferfluxCudaDispatchPhaseName(InferfluxCudaDispatchPhase phase) {
  switch (phase) {
  case InferfluxCudaDispatchPhase::kDecode: return "decode";
  case InferfluxCudaDispatchPhase::kPrefill: return "prefill";
  default: return "unknown";
  }
}

InferfluxCudaDispatchPhase ParseInferfluxCudaDispatchPhase(std::string_view phase) {
  if (phase == "decode") return InferfluxCudaDispatchPhase::kDecode;
  if (phase == "prefill") return InferfluxCudaDispatchPhase::kPrefill;
  return InferfluxCudaDispatchPhase::kUnknown;
}

InferfluxCudaDispatchBucket BucketBatchRows(int rows) {
  if (rows <= 1) return InferfluxCudaDispatchBucket::k1;
  if (rows == 2) return InferfluxCudaDispatchBucket::k2;
  if (rows <= 4) return InferfluxCudaDispatchBucket::k3_4;
  if (rows <= 8) return InferfluxCudaDispatchBucket::k5_8;
  if (rows <= 16) return InferfluxCudaDispatchBucket::k9_16;
  return InferfluxCudaDispatchBucket::k17Plus;
}

InferfluxCudaDispatchBucket BucketExtent(int extent) { return BucketBatchRows(extent); }

const char *InferfluxCudaDispatchBucketName(InferfluxCudaDispatchBucket bucket) {
  switch (bucket) {
  case InferfluxCudaDispatchBucket::k1: return "1";
  case InferfluxCudaDispatchBucket::k2: return "2";
  case InferfluxCudaDispatchBucket::k3_4: return "3_4";
  case InferfluxCudaDispatchBucket::k5_8: return "5_8";
  case InferfluxCudaDispatchBucket::k9_16: return "9_16";
  default: return "17_plus";
  }
}

InferfluxCudaFfnDispatchProfile BuildInferfluxCudaFfnDispatchProfile(
    InferfluxCudaDispatchPhase phase, int quant_type0, int quant_type1,
    const FusedDispatchGeometry &geometry, bool q81_ready, bool packed_ready) {
  Ffn p;
  p.phase = phase;
  p.quant_type0 = quant_type0;
  p.quant_type1 = quant_type1;
  p.geometry = geometry;
  p.same_quant = quant_type0 == quant_type1;
  p.q81_ready = q81_ready;
  p.packed_ready = packed_ready;
  p.m_bucket = BucketBatchRows(geometry.M);
  p.n_bucket = BucketExtent(geometry.N);
  p.k_bucket = BucketExtent(geometry.K);
  return p;
}

InferfluxCudaFfnDispatchDecision SelectInferfluxCudaFfnDispatchDecision(
    const InferfluxCudaFfnDispatchProfile &profile, const NativeExecutionPolicy &policy) {
  for (const FfnRule &r : FfnRules()) {
    if ((r.needs_q81 && !profile.q81_ready) || (r.needs_packed && !profile.packed_ready)) continue;
    if (r.match(profile, policy)) return {r.op, r.reason};
  }
  return {};
}

std::string DescribeInferfluxCudaFfnDispatchDecision(const InferfluxCudaFfnDispatchProfile &p,
                                                     std::string_view reason) {
  std::string s = "phase=";
  s += InferfluxCudaDispatchPhaseName(p.phase);
  s += ", quant0=" + TypeLabel(p.quant_type0) + ", quant1=" + TypeLabel(p.quant_type1);
  s += std::string(", q81_ready=") + Flag(p.q81_ready) + ", packed_ready=" + Flag(p.packed_ready);
  s += std::string(", m_bucket=") + InferfluxCudaDispatchBucketName(p.m_bucket) +
       ", n_bucket=" + InferfluxCudaDispatchBucketName(p.n_bucket) +
       ", k_bucket=" + InferfluxCudaDispatchBucketName(p.k_bucket);
  if (!reason.empty()) s += ", rule=" + std::string(reason);
  return s;
}

InferfluxCudaDownProjDispatchProfile BuildInferfluxCudaDownProjDispatchProfile(
    InferfluxCudaDispatchPhase phase, int quant_type, const FusedDispatchGeometry &geometry,
    bool q81_ready, bool packed_ready, bool mmq_ready) {
  Down p;
  p.phase = phase;
  p.quant_type = quant_type;
  p.geometry = geometry;
  p.q81_ready = q81_ready;
  p.packed_ready = packed_ready;
  p.mmq_ready = mmq_ready;
  p.m_bucket = BucketBatchRows(geometry.M);
  p.n_bucket = BucketExtent(geometry.N);
  p.k_bucket = BucketExtent(geometry.K);
  return p;
}

InferfluxCudaDownProjDispatchDecision SelectInferfluxCudaDownProjDispatchDecision(
    const InferfluxCudaDownProjDispatchProfile &profile, const NativeExecutionPolicy &policy) {
  for (const DownRule &r : DownRules()) {
    if ((r.needs_q81 && !profile.q81_ready) || (r.needs_packed && !profile.packed_ready) ||
        (r.needs_mmq && !profile.mmq_ready))
      continue;
    if (r.match(profile, policy)) return {r.op, r.reason};
  }
  return {};
}

std::string DescribeInferfluxCudaDownProjDispatchDecision(
    const InferfluxCudaDownProjDispatchProfile &p, std::string_view reason) {
  std::string s = "phase=";
  s += InferfluxCudaDispatchPhaseName(p.phase);
  s += ", quant=" + TypeLabel(p.quant_type);
  s += std::string(", q81_ready=") + Flag(p.q81_ready) + ", packed_ready=" + Flag(p.packed_ready) +
       ", mmq_ready=" + Flag(p.mmq_ready);
  s += std::string(", m_bucket=") + InferfluxCudaDispatchBucketName(p.m_bucket) +
       ", n_bucket=" + InferfluxCudaDispatchBucketName(p.n_bucket) +
       ", k_bucket=" + InferfluxCudaDispatchBucketName(p.k_bucket);
  if (!reason.empty()) s += ", rule=" + std::string(reason);
  return s;
}

// ---- native_dispatch_policy.cpp ----

const NativeExecutionPolicy &ResolveInferfluxCudaExecutionPolicy(
    const NativeExecutionPolicy *policy) {
  if (policy) return *policy;
  static thread_local NativeExecutionPolicy env_policy;
  env_policy = NativeExecutionPolicy::FromEnv();
  return env_policy;
}

std::string ProjectionQuantLabel(const QuantizedWeightInfo &weight) {
  return weight.data ? TypeLabel(weight.quant_type) : "unknown";
}

std::string ProjectionGroupQuantLabel(const QuantizedWeightInfo &first,
                                      const QuantizedWeightInfo &second) {
  if (!first.data || !second.data) return "unknown";
  return first.quant_type == second.quant_type ? ProjectionQuantLabel(first) : "mixed";
}

bool ForceCublasRequested(const NativeExecutionPolicy &policy) { return policy.force_cublas; }
bool PackedActivationsDisabled(const NativeExecutionPolicy &policy) {
  return policy.disable_prepacked_activations;
}
bool Q81ActivationsDisabled(const NativeExecutionPolicy &policy) {
  return policy.disable_q81_activations;
}

// native_dispatch_policy.cpp:46-72: a fused kernel exists for the
// projection (the policy's activation switches choose which one, so either
// answer past ShouldUseFusedPath is true).
bool ProjectionHasGraphSafeKernel(const QuantizedWeightInfo &raw,
                                  const FusedDispatchGeometry &geometry,
                                  bool allow_fused_quantized_matmul,
                                  const NativeExecutionPolicy &policy) {
  if (ForceCublasRequested(policy) || !allow_fused_quantized_matmul || !raw.data ||
      raw.quant_type < 0 || geometry.M <= 0 || geometry.N <= 0 || geometry.K <= 0)
    return false;
  return FusedQuantGemm::ShouldUseFusedPath(raw.quant_type, geometry);
}

namespace {

bool ReadyForSingle(int quant_type, const FusedDispatchGeometry &g, bool supported) {
  const FusedDispatchGeometry single{g.M, g.N, g.K, 1, true, false};
  return supported && FusedQuantGemm::ShouldUseFusedPath(quant_type, single);
}

bool MmqReady(int quant_type, const FusedDispatchGeometry &g) {
  return FusedQuantGemm::SupportsDownProjMmq(quant_type) &&
         g.M >= FusedQuantGemm::GetDownProjMmqThreshold(quant_type, g.M, g.N, g.K) &&
         g.M <= FusedQuantGemm::kDownProjMmqMaxM;
}

}  // namespace

FusedQuantGemm::DownProjOperator SelectInferfluxCudaDownProjOperator(
    const QuantizedWeightInfo &raw, const MmqWeightInfo &mmq_weight,
    InferfluxCudaDispatchPhase phase, const FusedDispatchGeometry &geometry,
    bool allow_fused_quantized_matmul, const NativeExecutionPolicy &policy) {
  if (ForceCublasRequested(policy) || !allow_fused_quantized_matmul) return DownOp::kFallback;
  const bool q81 = ReadyForSingle(raw.quant_type, geometry,
                                  !Q81ActivationsDisabled(policy) &&
                                      FusedQuantGemm::SupportsQ8_1Activations(raw.quant_type));
  const bool packed =
      ReadyForSingle(raw.quant_type, geometry,
                     !PackedActivationsDisabled(policy) &&
                         FusedQuantGemm::SupportsPackedActivations(raw.quant_type));
  const bool mmq = mmq_weight.data != nullptr && FusedQuantGemm::IsDownProjMmqEnabled(&policy) &&
                   MmqReady(raw.quant_type, geometry);
  const auto profile =
      BuildInferfluxCudaDownProjDispatchProfile(phase, raw.quant_type, geometry, q81, packed, mmq);
  return SelectInferfluxCudaDownProjDispatchDecision(profile, policy).op;
}

FusedQuantGemm::FfnProjOperator SelectInferfluxCudaFfnProjOperator(
    const QuantizedWeightInfo &gate_raw, const QuantizedWeightInfo &up_raw,
    InferfluxCudaDispatchPhase phase, const FusedDispatchGeometry &geometry,
    bool allow_fused_quantized_matmul, const NativeExecutionPolicy &policy) {
  if (ForceCublasRequested(policy) || !allow_fused_quantized_matmul) return FfnOp::kFallback;
  const FusedDispatchGeometry single{geometry.M, geometry.N, geometry.K, 1,
                                     geometry.packed_activation, geometry.includes_rmsnorm};
  const auto ok = [&](int t) { return FusedQuantGemm::ShouldUseFusedPath(t, single); };
  const bool q81 = !Q81ActivationsDisabled(policy) &&
                   FusedQuantGemm::SupportsQ8_1Activations(gate_raw.quant_type) &&
                   FusedQuantGemm::SupportsQ8_1Activations(up_raw.quant_type) &&
                   ok(gate_raw.quant_type) && ok(up_raw.quant_type);
  const bool packed = !PackedActivationsDisabled(policy) &&
                      FusedQuantGemm::SupportsPackedActivations(gate_raw.quant_type) &&
                      FusedQuantGemm::SupportsPackedActivations(up_raw.quant_type) &&
                      ok(gate_raw.quant_type) && ok(up_raw.quant_type);
  const auto profile = BuildInferfluxCudaFfnDispatchProfile(phase, gate_raw.quant_type,
                                                            up_raw.quant_type, geometry, q81,
                                                            packed);
  return SelectInferfluxCudaFfnDispatchDecision(profile, policy).op;
}

// ---- FusedQuantGemm selectors (fused_quant_gemm.cu:945-1128) ----

bool FusedQuantGemm::ShouldUseSpecializedQ8_1GroupedFastPath(int quant_type,
                                                             const FusedDispatchGeometry &g,
                                                             const NativeExecutionPolicy *policy) {
  return ResolveInferfluxCudaExecutionPolicy(policy).enable_experimental_q81_grouped_hot_q4k &&
         quant_type == kQ4K && g.grouped_outputs == 2 && g.M == 1 && g.N >= 8192 &&
         g.K == kGroupedHotK;
}

bool FusedQuantGemm::ShouldUseSpecializedQ8_1GroupedRowPairW4Path(
    int quant_type, const FusedDispatchGeometry &g, const NativeExecutionPolicy *policy) {
  return ResolveInferfluxCudaExecutionPolicy(policy).enable_experimental_q81_grouped_rowpair_w4 &&
         quant_type == kQ4K && g.grouped_outputs == 2 && g.M == 2 && g.N >= 8192 &&
         g.K == kGroupedHotK;
}

bool FusedQuantGemm::ShouldUseSpecializedQ8_1DownProjHotPath(int quant_type,
                                                             const FusedDispatchGeometry &g,
                                                             const NativeExecutionPolicy *) {
  return Q4KOrQ6K(quant_type) && g.grouped_outputs == 1 && g.M == 1 && g.N == kDownHotN &&
         g.K == kDownHotK;
}

bool FusedQuantGemm::ShouldUseSpecializedQ8_1DownProjRowPairHotPath(
    int quant_type, const FusedDispatchGeometry &g, const NativeExecutionPolicy *) {
  return Q4KOrQ6K(quant_type) && g.grouped_outputs == 1 && g.M == 2 && g.N == kDownHotN &&
         g.K == kDownHotK;
}

FusedQuantGemm::FfnProjOperator FusedQuantGemm::SelectFfnProjOperator(
    int quant_type0, int quant_type1, const FusedDispatchGeometry &geometry, bool allow_q81,
    bool allow_packed, const NativeExecutionPolicy *policy) {
  const NativeExecutionPolicy &pol = ResolveInferfluxCudaExecutionPolicy(policy);
  if (geometry.M <= 0 || geometry.N <= 0 || geometry.K <= 0 || geometry.grouped_outputs != 2)
    return FfnOp::kFallback;
  const FusedDispatchGeometry single{geometry.M, geometry.N, geometry.K, 1,
                                     geometry.packed_activation, geometry.includes_rmsnorm};
  const bool fits = ShouldUseFusedPath(quant_type0, single) && ShouldUseFusedPath(quant_type1, single);
  const bool q81 = allow_q81 && SupportsQ8_1Activations(quant_type0) &&
                   SupportsQ8_1Activations(quant_type1) && fits;
  const bool packed = allow_packed && SupportsPackedActivations(quant_type0) &&
                      SupportsPackedActivations(quant_type1) && fits;
  const auto profile = BuildInferfluxCudaFfnDispatchProfile(
      InferfluxCudaDispatchPhase::kDecode, quant_type0, quant_type1, geometry, q81, packed);
  return SelectInferfluxCudaFfnDispatchDecision(profile, pol).op;
}

const char *FusedQuantGemm::FfnProjOperatorName(FfnProjOperator op) {
  switch (op) {
  case FfnOp::kQ81Group: return "q8_1_group";
  case FfnOp::kQ81GroupHotQ4K: return "q8_1_group_hot_q4k";
  case FfnOp::kQ81GroupRowPairW4: return "q8_1_group_row_pair_w4";
  case FfnOp::kQ81GroupRowQuadM4: return "q8_1_group_row_quad_m4";
  case FfnOp::kQ81GroupMmq3: return "q8_1_group_mmq3";
  case FfnOp::kPackedGroup: return "packed_group";
  default: return "fallback";
  }
}

const char *FusedQuantGemm::FfnProjOperatorMetricName(FfnProjOperator op, int quant_type, int m,
                                                      int k) {
  (void)k;
  if (op == FfnOp::kQ81Group && Q4KOrQ6K(quant_type))
    return m <= 8 ? "q8_1_group_mmvq" : "q8_1_group_mmq";
  return FfnProjOperatorName(op);
}

FusedQuantGemm::DownProjOperator FusedQuantGemm::SelectDownProjOperator(
    int quant_type, const FusedDispatchGeometry &geometry, bool allow_q81, bool allow_packed,
    bool allow_mmq, const NativeExecutionPolicy *policy) {
  const NativeExecutionPolicy &pol = ResolveInferfluxCudaExecutionPolicy(policy);
  if (geometry.M <= 0 || geometry.N <= 0 || geometry.K <= 0) return DownOp::kFallback;
  const bool q81 = ReadyForSingle(quant_type, geometry, allow_q81 && SupportsQ8_1Activations(quant_type));
  const bool packed =
      ReadyForSingle(quant_type, geometry, allow_packed && SupportsPackedActivations(quant_type));
  const bool mmq = allow_mmq && MmqReady(quant_type, geometry);
  const auto profile = BuildInferfluxCudaDownProjDispatchProfile(
      InferfluxCudaDispatchPhase::kUnknown, quant_type, geometry, q81, packed, mmq);
  return SelectInferfluxCudaDownProjDispatchDecision(profile, pol).op;
}

const char *FusedQuantGemm::DownProjOperatorName(DownProjOperator op) {
  switch (op) {
  case DownOp::kQ81Gemv: return "q8_1_gemv";
  case DownOp::kQ81GemvHotFixed: return "q8_1_gemv_hot_fixed";
  case DownOp::kQ81GemvRowPairHotFixed: return "q8_1_gemv_row_pair_hot_fixed";
  case DownOp::kQ81GemvRowPair: return "q8_1_gemv_row_pair";
  case DownOp::kQ81GemvRowQuad: return "q8_1_gemv_row_quad";
  case DownOp::kPackedGemv: return "packed_gemv";
  case DownOp::kMmq: return "mmq";
  default: return "fallback";
  }
}

const char *FusedQuantGemm::DownProjOperatorMetricName(DownProjOperator op, int quant_type, int m,
                                                       int k) {
  (void)quant_type;
  (void)k;
  if (op == DownOp::kQ81Gemv) return m <= 8 ? "q8_1_mmvq" : "q8_1_mmq";
  return DownProjOperatorName(op);
}

}  // namespace rocm
}  // namespace inferflux
