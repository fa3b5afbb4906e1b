// fused_quant_gemm.cpp -- C++ host mirror of InferFlux's FusedQuantGemm
// (runtime/backends/cuda/native/fused_quant_gemm.cu) over the gfx950 C ABI
// (include/ifx_qgemm.h).  It carries the reference's host conventions --
// bool "launched" results, QuantizedWeightInfo views, the
// INFERFLUX_DISABLE_FUSED_GEMV policy switch -- and leaves every launch to
// the C ABI, which validates arguments and reports HIP errors.
#include <algorithm>
#include "../../include/ifx_fused_quant_gemm.h"

#include <cstdlib>
#include <cstring>

#include "../../include/ifx_qgemm.h"

namespace inferflux {
namespace rocm {

namespace {

// Policy resolution (fused_quant_gemm.cu:28-42): an explicit policy wins,
// else the environment, read on each call as the reference does.
NativeExecutionPolicy Resolve(const NativeExecutionPolicy *policy) {
  return policy ? *policy : NativeExecutionPolicy::FromEnv();
}

bool ParseBoolEnv(const char *name, bool fallback) {
  const char *v = std::getenv(name);
  if (!v || !*v) return fallback;
  if (!std::strcmp(v, "1") || !strcasecmp(v, "true") || !strcasecmp(v, "yes") ||
      !strcasecmp(v, "on"))
    return true;
  if (!std::strcmp(v, "0") || !strcasecmp(v, "false") || !strcasecmp(v, "no") ||
      !strcasecmp(v, "off"))
    return false;
  return fallback;
}

// string_utils.h:55-68: the fallback when unset, empty, unparseable or
// outside [lo, hi].
int ParseIntEnv(const char *name, int fallback, int lo, int hi) {
  const char *v = std::getenv(name);
  if (!v || !*v) return fallback;
  char *end = nullptr;
  const long n = std::strtol(v, &end, 10);
  if (end == v || *end != '\0' || n < lo || n > hi) return fallback;
  return static_cast<int>(n);
}

bool Usable(const QuantizedWeightInfo &w, const void *act, const void *out) {
  return w.data && w.quant_type >= 0 && act && out;
}

// The view must hold at least N x K elements when its size is known.
bool ViewCovers(const QuantizedWeightInfo &w, int N, int K) {
  return w.num_elements <= 0 ||
         w.num_elements >= static_cast<int64_t>(N) * static_cast<int64_t>(K);
}

// Which entry a launch takes.  need: the ordered workspace bytes of the
// launch through the ordered entries (0: it does not split there).  With
// deterministic_reductions the ordered entry is required (a split without a
// large enough workspace: not handled); without it, a caller-given
// reduction_workspace selects the ordered entry too when it fits (size and
// 256-byte alignment) or is not needed, and anything else takes the plain
// entry, whose K splits add with fp32 atomics (the plain entry may also
// split launches the ordered entry runs unsplit: fp32 accumulate at
// 9 <= M <= 16).
enum class Reduction { kAtomic, kOrdered, kRefuse };
Reduction SplitReduction(const NativeExecutionPolicy &p, int64_t need) {
  if (need <= 0)
    return p.deterministic_reductions || p.reduction_workspace ? Reduction::kOrdered
                                                               : Reduction::kAtomic;
  const bool fits = p.reduction_workspace && p.reduction_workspace_bytes >= need &&
                    reinterpret_cast<uintptr_t>(p.reduction_workspace) % 256 == 0;
  if (fits) return Reduction::kOrdered;
  return p.deterministic_reductions ? Reduction::kRefuse : Reduction::kAtomic;
}

bool Launch(const QuantizedWeightInfo &w, const void *act, void *out, int out_dtype, int mode,
            const void *bias, int M, int N, int K, hipStream_t stream,
            const NativeExecutionPolicy *policy) {
  if (!Usable(w, act, out)) return false;
  if (Resolve(policy).disable_fused_gemv) return false;
  if (!ViewCovers(w, N, K)) return false;
  const FusedDispatchGeometry g{M, N, K, 1, true, false};
  if (!FusedQuantGemm::ShouldUseFusedPath(w.quant_type, g)) return false;
  const NativeExecutionPolicy p = Resolve(policy);
  switch (SplitReduction(p, ifx_qgemv_workspace_bytes(w.quant_type, 1, &N, out_dtype, M, K))) {
  case Reduction::kRefuse: return false;
  case Reduction::kOrdered:
    return ifx_qgemv_ws(w.quant_type, w.data, act, out, out_dtype, mode, bias, M, N, K,
                        p.reduction_workspace,
                        p.reduction_workspace ? p.reduction_workspace_bytes : 0, stream) == IFX_OK;
  case Reduction::kAtomic: break;
  }
  return ifx_qgemv(w.quant_type, w.data, act, out, out_dtype, mode, bias, M, N, K, stream) ==
         IFX_OK;
}

template <size_t C>
bool LaunchGroup(const std::array<PackedProjectionSpec, C> &p, const void *act, int M, int K,
                 hipStream_t stream, const NativeExecutionPolicy *policy) {
  if (!act || Resolve(policy).disable_fused_gemv) return false;
  const void *W[C];
  void *Y[C];
  int N[C];
  for (size_t i = 0; i < C; ++i) {
    if (!Usable(p[i].weight, act, p[i].output)) return false;
    if (p[i].weight.quant_type != p[0].weight.quant_type) return false;
    if (!ViewCovers(p[i].weight, p[i].output_cols, K)) return false;
    W[i] = p[i].weight.data;
    Y[i] = p[i].output;
    N[i] = p[i].output_cols;
  }
  const FusedDispatchGeometry g{M, N[0], K, static_cast<int>(C), true, false};
  if (!FusedQuantGemm::ShouldUseFusedPath(p[0].weight.quant_type, g)) return false;
  const NativeExecutionPolicy pol = Resolve(policy);
  switch (SplitReduction(pol, ifx_qgemv_workspace_bytes(p[0].weight.quant_type,
                                                        static_cast<int>(C), N, IFX_OUT_F16, M,
                                                        K))) {
  case Reduction::kRefuse: return false;
  case Reduction::kOrdered:
    return ifx_qgemv_grouped_ws(p[0].weight.quant_type, static_cast<int>(C), W, Y, N, act,
                                IFX_OUT_F16, IFX_STORE, M, K, pol.reduction_workspace,
                                pol.reduction_workspace ? pol.reduction_workspace_bytes : 0,
                                stream) == IFX_OK;
  case Reduction::kAtomic: break;
  }
  return ifx_qgemv_grouped(p[0].weight.quant_type, static_cast<int>(C), W, Y, N, act,
                           IFX_OUT_F16, IFX_STORE, M, K, stream) == IFX_OK;
}

}  // namespace

// native_execution_policy.h:61-78: the same environment names and
// fallbacks, apart from INFERFLUX_ENABLE_DOWNPROJ_MMQ's default (the
// struct's comment says why).
NativeExecutionPolicy NativeExecutionPolicy::FromEnv() {
  NativeExecutionPolicy p;
  p.force_cublas = ParseBoolEnv("INFERFLUX_FORCE_CUBLAS", false);
  p.disable_prepacked_activations = ParseBoolEnv("INFERFLUX_DISABLE_PREPACKED_ACTIVATIONS", false);
  p.disable_q81_activations = ParseBoolEnv("INFERFLUX_DISABLE_Q8_1_ACTIVATIONS", false);
  p.disable_fused_gemv = ParseBoolEnv("INFERFLUX_DISABLE_FUSED_GEMV", false);
  p.enable_experimental_q81_downproj_hot_fixed =
      ParseBoolEnv("INFERFLUX_ENABLE_EXPERIMENTAL_Q8_1_DOWNPROJ_HOT_FIXED", false);
  p.enable_experimental_q81_downproj_rowpair_hot_fixed =
      ParseBoolEnv("INFERFLUX_ENABLE_EXPERIMENTAL_Q8_1_DOWNPROJ_ROWPAIR_HOT_FIXED", false);
  p.enable_experimental_q81_grouped_hot_q4k =
      ParseBoolEnv("INFERFLUX_ENABLE_EXPERIMENTAL_Q8_1_GROUPED_HOT_Q4K", true);
  p.enable_experimental_q81_grouped_rowpair_w4 =
      ParseBoolEnv("INFERFLUX_ENABLE_EXPERIMENTAL_Q8_1_GROUPED_ROWPAIR_W4", true);
  p.enable_experimental_q81_grouped_rowquad_m4 =
      ParseBoolEnv("INFERFLUX_ENABLE_EXPERIMENTAL_Q8_1_GROUPED_ROWQUAD_M4", false);
  p.enable_experimental_q81_grouped_mmq3 =
      ParseBoolEnv("INFERFLUX_ENABLE_EXPERIMENTAL_Q8_1_GROUPED_MMQ3", true);
  p.enable_downproj_mmq = ParseBoolEnv("INFERFLUX_ENABLE_DOWNPROJ_MMQ", true);
  p.downproj_mmq_min_batch_override = ParseIntEnv("INFERFLUX_DOWNPROJ_MMQ_MIN_BATCH", -1, 1, 64);
  p.enable_fused_gate_up_silu = ParseBoolEnv("INFERFLUX_ENABLE_FUSED_GATE_UP_SILU", true);
  return p;
}

void FusedQuantGemm::QuantizeRowQ8_1(const uint16_t *input, void *output_q8_1, int M, int K,
                                     hipStream_t stream) {
  ifx_q8_1_quantize_f16(input, output_q8_1, M, K, stream);
}

void FusedQuantGemm::QuantizeRowQ8_1(const float *input, void *output_q8_1, int M, int K,
                                     hipStream_t stream) {
  ifx_q8_1_quantize_f32(input, output_q8_1, M, K, stream);
}

void FusedQuantGemm::SiluMulQuantizeQ8_1(const uint16_t *gate, const uint16_t *up,
                                         void *output_q8_1, int M, int K, hipStream_t stream) {
  ifx_silu_mul_quantize_q8_1(gate, up, IFX_OUT_F16, output_q8_1, M, K, stream);
}

void FusedQuantGemm::SiluMulQuantizeQ8_1(const float *gate, const float *up, void *output_q8_1,
                                         int M, int K, hipStream_t stream) {
  ifx_silu_mul_quantize_q8_1(gate, up, IFX_OUT_F32, output_q8_1, M, K, stream);
}

void FusedQuantGemm::FusedRmsNormQuantizeQ8_1(const uint16_t *residual,
                                              const uint16_t *norm_weight, void *output_q8_1,
                                              int M, int K, float rms_norm_eps,
                                              hipStream_t stream) {
  ifx_rmsnorm_quantize_q8_1(residual, IFX_OUT_F16, norm_weight, output_q8_1, M, K, rms_norm_eps,
                            stream);
}

void FusedQuantGemm::FusedRmsNormQuantizeQ8_1(const float *residual, const uint16_t *norm_weight,
                                              void *output_q8_1, int M, int K,
                                              float rms_norm_eps, hipStream_t stream) {
  ifx_rmsnorm_quantize_q8_1(residual, IFX_OUT_F32, norm_weight, output_q8_1, M, K, rms_norm_eps,
                            stream);
}

bool FusedQuantGemm::GemvQ8_1(const QuantizedWeightInfo &weight, const void *act_q8_1,
                              uint16_t *output, int M, int N, int K, hipStream_t stream,
                              const NativeExecutionPolicy *policy) {
  return Launch(weight, act_q8_1, output, IFX_OUT_F16, IFX_STORE, nullptr, M, N, K, stream,
                policy);
}

bool FusedQuantGemm::GemvQ8_1F32(const QuantizedWeightInfo &weight, const void *act_q8_1,
                                 float *output, int M, int N, int K, hipStream_t stream,
                                 const NativeExecutionPolicy *policy) {
  return Launch(weight, act_q8_1, output, IFX_OUT_F32, IFX_STORE, nullptr, M, N, K, stream,
                policy);
}

bool FusedQuantGemm::GemvQ8_1Accum(const QuantizedWeightInfo &weight, const void *act_q8_1,
                                   uint16_t *output, int M, int N, int K, hipStream_t stream,
                                   const NativeExecutionPolicy *policy) {
  return Launch(weight, act_q8_1, output, IFX_OUT_F16, IFX_ACCUM, nullptr, M, N, K, stream,
                policy);
}

bool FusedQuantGemm::GemvQ8_1AccumF32(const QuantizedWeightInfo &weight, const void *act_q8_1,
                                      float *output, int M, int N, int K, hipStream_t stream,
                                      const NativeExecutionPolicy *policy) {
  return Launch(weight, act_q8_1, output, IFX_OUT_F32, IFX_ACCUM, nullptr, M, N, K, stream,
                policy);
}

bool FusedQuantGemm::GemvQ8_1WithBias(const QuantizedWeightInfo &weight, const void *act_q8_1,
                                      uint16_t *output, const uint16_t *bias, int M, int N,
                                      int K, hipStream_t stream,
                                      const NativeExecutionPolicy *policy) {
  return Launch(weight, act_q8_1, output, IFX_OUT_F16, bias ? IFX_BIAS : IFX_STORE, bias, M, N,
                K, stream, policy);
}

bool FusedQuantGemm::GemvQ8_1Pair(const std::array<PackedProjectionSpec, 2> &projections,
                                  const void *act_q8_1, int M, int K, hipStream_t stream,
                                  const NativeExecutionPolicy *policy,
                                  FfnProjOperator selected_op) {
  // Every label runs the routed grouped launch; an out-of-range value is a
  // caller error and is not handled.
  if (static_cast<int>(selected_op) < static_cast<int>(FfnProjOperator::kFallback) ||
      static_cast<int>(selected_op) > static_cast<int>(FfnProjOperator::kPackedGroup))
    return false;
  return LaunchGroup(projections, act_q8_1, M, K, stream, policy);
}

bool FusedQuantGemm::GemvQ8_1PairRowQuadCandidate(
    const std::array<PackedProjectionSpec, 2> &projections, const void *act_q8_1, int M, int K,
    hipStream_t stream) {
  return LaunchGroup(projections, act_q8_1, M, K, stream, nullptr);
}

bool FusedQuantGemm::GemvQ8_1Triple(const std::array<PackedProjectionSpec, 3> &projections,
                                    const void *act_q8_1, int M, int K, hipStream_t stream,
                                    const NativeExecutionPolicy *policy) {
  return LaunchGroup(projections, act_q8_1, M, K, stream, policy);
}

bool FusedQuantGemm::FusedGateUpSiluGemvQ8_1(const QuantizedWeightInfo &gate_raw,
                                             const QuantizedWeightInfo &up_raw,
                                             const void *act_q8_1, uint16_t *output, int M,
                                             int N, int K, hipStream_t stream) {
  return FusedGateUpSiluGemvQ8_1WithEpilogue(gate_raw, up_raw, act_q8_1, output, nullptr, M, N, K,
                                             stream);
}

bool FusedQuantGemm::FusedGateUpSiluGemvQ8_1WithEpilogue(const QuantizedWeightInfo &gate_raw,
                                                         const QuantizedWeightInfo &up_raw,
                                                         const void *act_q8_1, uint16_t *output,
                                                         void *act_q8_1_out, int M, int N, int K,
                                                         hipStream_t stream) {
  if (!Usable(gate_raw, act_q8_1, output) || !Usable(up_raw, act_q8_1, output)) return false;
  if (gate_raw.quant_type != up_raw.quant_type) return false;
  if (!ViewCovers(gate_raw, N, K) || !ViewCovers(up_raw, N, K)) return false;
  return ifx_qgemv_gate_up_silu(gate_raw.quant_type, gate_raw.data, up_raw.data, act_q8_1, output,
                                IFX_OUT_F16, act_q8_1_out, M, N, K, stream) == IFX_OK;
}

namespace {

template <size_t C>
bool LaunchPacked(const std::array<PackedProjectionSpec, C> &p, const PackedActivationInfo &act,
                  int M, int K, hipStream_t stream, const NativeExecutionPolicy *policy) {
  if (!act.data || !act.row_scales || M <= 0 || Resolve(policy).disable_fused_gemv) return false;
  if (!FusedQuantGemm::SupportsPackedActivations(p[0].weight.quant_type)) return false;
  const void *W[C];
  void *Y[C];
  int N[C];
  for (size_t i = 0; i < C; ++i) {
    if (!Usable(p[i].weight, act.data, p[i].output) || p[i].output_cols <= 0) return false;
    if (p[i].weight.quant_type != p[0].weight.quant_type) return false;
    if (!ViewCovers(p[i].weight, p[i].output_cols, K)) return false;
    W[i] = p[i].weight.data;
    Y[i] = p[i].output;
    N[i] = p[i].output_cols;
  }
  return ifx_qgemv_packed(p[0].weight.quant_type, static_cast<int>(C), W, Y, N, act.data,
                          act.row_scales, M, K, stream) == IFX_OK;
}

}  // namespace

bool FusedQuantGemm::GemvPacked(const QuantizedWeightInfo &weight,
                                const PackedActivationInfo &activation, uint16_t *output, int M,
                                int N, int K, hipStream_t stream,
                                const NativeExecutionPolicy *policy) {
  const std::array<PackedProjectionSpec, 1> p{PackedProjectionSpec{weight, output, N}};
  return LaunchPacked(p, activation, M, K, stream, policy);
}

bool FusedQuantGemm::GemvPackedPair(const std::array<PackedProjectionSpec, 2> &projections,
                                    const PackedActivationInfo &activation, int M, int K,
                                    hipStream_t stream) {
  return LaunchPacked(projections, activation, M, K, stream, nullptr);
}

bool FusedQuantGemm::GemvPackedTriple(const std::array<PackedProjectionSpec, 3> &projections,
                                      const PackedActivationInfo &activation, int M, int K,
                                      hipStream_t stream) {
  return LaunchPacked(projections, activation, M, K, stream, nullptr);
}

bool FusedQuantGemm::SupportsPackedActivations(int quant_type) {
  return quant_type == static_cast<int>(TensorType::Q4_K) ||
         quant_type == static_cast<int>(TensorType::Q6_K) ||
         quant_type == static_cast<int>(TensorType::Q8_0) ||
         quant_type == static_cast<int>(TensorType::Q8_K);
}

bool FusedQuantGemm::QuantizeRowsSymmetric(const uint16_t *input, int8_t *output,
                                           float *row_scales, int rows, int cols,
                                           hipStream_t stream) {
  return ifx_quantize_rows_symmetric(input, IFX_OUT_F16, output, row_scales, rows, cols,
                                     stream) == IFX_OK;
}

bool FusedQuantGemm::SiluMulQuantizeRowsSymmetric(const uint16_t *gate, const uint16_t *up,
                                                  int8_t *output, float *row_scales, int rows,
                                                  int cols, hipStream_t stream) {
  return ifx_silu_mul_quantize_rows_symmetric(gate, up, IFX_OUT_F16, output, row_scales, rows,
                                              cols, stream) == IFX_OK;
}

bool FusedQuantGemm::SupportsQ8_1Activations(int quant_type) {
  return quant_type == static_cast<int>(TensorType::Q4_K) ||
         quant_type == static_cast<int>(TensorType::Q5_K) ||
         quant_type == static_cast<int>(TensorType::Q6_K) ||
         quant_type == static_cast<int>(TensorType::Q8_0) ||
         quant_type == static_cast<int>(TensorType::Q8_K);
}

// The reference scales a per-GPU-generation base by 16/bpw and clamps to
// [4, 64] (fused_quant_gemm.cu:62-184, 830-880): above it, dequantize +
// FP16 cuBLAS wins on its tensor cores.  On gfx950 the quantized path itself
// switches to an fp16 MFMA GEMM that dequantizes inside the kernel (from
// M = 33 for Q6_K, 96 for Q4_K, 128 for Q8_0; below that the integer-dot
// kernels), which reads the raw blocks instead of an FP16 copy and measured
// 1.4-1.7x faster than dequantize + the vendor FP16 GEMM at the 32B prefill
// shapes, so the fallback never wins: the threshold is the path's M limit.
int FusedQuantGemm::GetAdaptiveThreshold(int quant_type) {
  if (!SupportsQ8_1Activations(quant_type)) return 0;
  if (quant_type == static_cast<int>(TensorType::Q5_K) ||
      quant_type == static_cast<int>(TensorType::Q8_K))
    return kMaxGemvOnlyM;  // v_dot4 GEMV only
  return kMaxFusedM;
}

// The geometry narrows it where a kernel has a hard limit (the reference
// adjusts its threshold for packed activations, grouped outputs and K,
// fused_quant_gemm.cu:830-923; like it, includes_rmsnorm counts only when
// the activations are not pre-quantized, packed_activation == false):
//  * includes_rmsnorm without pre-quantized activations: the RMSNorm + Q8_1
//    producer fused into the GEMV (ifx_qgemv_grouped_rmsnorm) is Q4_K only,
//    M <= 2, with the batch's Q8_1 rows (80 K / 64 + K / 8 bytes each) in
//    64 KiB of LDS; larger batches take the producer + GEMV;
//  * K: the Q8_1 activations [M][K/32] are addressed with 32-bit offsets.
int FusedQuantGemm::GetGeometryAwareThreshold(int quant_type,
                                              const FusedDispatchGeometry &geometry) {
  int64_t t = GetAdaptiveThreshold(quant_type);
  if (t == 0) return 0;
  const int64_t a_row = geometry.K > 0 ? static_cast<int64_t>(geometry.K / 32) * 36 : 0;
  if (geometry.includes_rmsnorm && !geometry.packed_activation) {
    if (quant_type != static_cast<int>(TensorType::Q4_K)) return 0;
    t = std::min<int64_t>(t, 2);
    // the LDS row of the fused producer: codes in 80-byte slots per 64
    // values, then 4 bytes of d | s per block of 32
    const int64_t lds_row = geometry.K > 0 ? static_cast<int64_t>(geometry.K / 64) * 80 + geometry.K / 8 : 0;
    if (lds_row > 0) t = std::min<int64_t>(t, 65536 / lds_row);
  }
  if (a_row > 0) t = std::min<int64_t>(t, ((int64_t{1} << 32) - 1) / a_row);
  return static_cast<int>(t);
}

bool FusedQuantGemm::ShouldUseFusedPath(int quant_type, int M) {
  const FusedDispatchGeometry geometry{M, 0, 0, 1, false, false};
  return ShouldUseFusedPath(quant_type, geometry);
}

bool FusedQuantGemm::ShouldUseFusedPath(int quant_type, const FusedDispatchGeometry &geometry) {
  if (geometry.M <= 0) return false;
  if (geometry.grouped_outputs < 1 || geometry.grouped_outputs > 3) return false;
  if (!SupportsQ8_1Activations(quant_type)) return false;
  if (geometry.M > GetGeometryAwareThreshold(quant_type, geometry)) return false;
  // Known N and K must fit the kernels (K a whole number of blocks, 32-bit
  // byte offsets); unknown (0) ones are decided at launch.
  if (geometry.N > 0 && geometry.K > 0)
    return ifx_supports(quant_type, geometry.M, geometry.N, geometry.K) != 0;
  return true;
}

KernelFamily FusedQuantGemm::SelectKernel(int quant_type, int M, int N, int K) {
  return static_cast<KernelFamily>(ifx_kernel_family(quant_type, M, N, K));
}

const char *FusedQuantGemm::KernelFamilyName(KernelFamily family) {
  switch (family) {
  case KernelFamily::kGemv: return "v_dot4 GEMV";
  case KernelFamily::kSkinnyMfma: return "skinny int8 MFMA";
  case KernelFamily::kTiledMfma: return "tiled int8 MFMA";
  case KernelFamily::kF16DequantMfma: return "fp16 MFMA, in-kernel dequant";
  case KernelFamily::kF16DequantGemv: return "fp16 dequant MFMA GEMV";
  default: return "none";
  }
}

// ---- Down projection on the re-tiled copy ----

namespace {

bool DownProjLaunch(const MmqWeightInfo &w, const void *act, void *out, int out_dtype, int mode,
                    int M, int N, int K, hipStream_t stream, const NativeExecutionPolicy *policy) {
  const NativeExecutionPolicy p = Resolve(policy);
  if (!p.enable_downproj_mmq || p.disable_fused_gemv) return false;
  if (!w.data || !act || !out || M <= 0 || N <= 0 || K <= 0) return false;
  if (N != w.rows || K != w.cols || w.tile_cols != FusedQuantGemm::kDownProjMmqTileCols)
    return false;
  if (!FusedQuantGemm::SupportsDownProjMmq(w.quant_type) || M > FusedQuantGemm::kDownProjMmqMaxM)
    return false;
  return ifx_qgemv_mmq(w.quant_type, w.data, act, out, out_dtype, mode, M, N, K,
                       p.deterministic_reductions ? 1 : 0, stream) == IFX_OK;
}

}  // namespace

bool FusedQuantGemm::DownProjMmq(const MmqWeightInfo &weight, const void *act_q8_1,
                                 uint16_t *output, int M, int N, int K, hipStream_t stream,
                                 const NativeExecutionPolicy *policy) {
  return DownProjLaunch(weight, act_q8_1, output, IFX_OUT_F16, IFX_STORE, M, N, K, stream, policy);
}

bool FusedQuantGemm::DownProjMmqF32(const MmqWeightInfo &weight, const void *act_q8_1,
                                    float *output, int M, int N, int K, hipStream_t stream,
                                    const NativeExecutionPolicy *policy) {
  return DownProjLaunch(weight, act_q8_1, output, IFX_OUT_F32, IFX_STORE, M, N, K, stream, policy);
}

bool FusedQuantGemm::DownProjMmqAccumF32(const MmqWeightInfo &weight, const void *act_q8_1,
                                         float *output, int M, int N, int K, hipStream_t stream,
                                         const NativeExecutionPolicy *policy) {
  return DownProjLaunch(weight, act_q8_1, output, IFX_OUT_F32, IFX_ACCUM, M, N, K, stream, policy);
}

bool FusedQuantGemm::IsDownProjMmqEnabled(const NativeExecutionPolicy *policy) {
  return Resolve(policy).enable_downproj_mmq;
}

// fused_quant_gemm.cu:1966-2026: validate, allocate, transform on the
// stream, wait, and hand the caller the layout (freed on any failure).
bool FusedQuantGemm::BuildDownProjMmqLayout(const QuantizedWeightInfo &weight, int rows, int cols,
                                            MmqWeightInfo *layout, hipStream_t stream) {
  if (!layout || !weight.data || rows <= 0 || cols <= 0 || cols % 256 != 0) return false;
  if (!SupportsDownProjMmq(weight.quant_type)) return false;
  if (!ViewCovers(weight, rows, cols)) return false;
  const int64_t bytes = ifx_mmq_layout_bytes(weight.quant_type, rows, cols);
  if (bytes <= 0) return false;
  void *buf = nullptr;
  if (hipMalloc(&buf, static_cast<size_t>(bytes)) != hipSuccess) return false;
  if (ifx_mmq_layout_build(weight.quant_type, weight.data, buf, rows, cols, stream) != IFX_OK ||
      hipStreamSynchronize(stream) != hipSuccess) {
    (void)hipFree(buf);
    return false;
  }
  *layout = MmqWeightInfo{buf, weight.quant_type, rows, cols, kDownProjMmqTileCols};
  return true;
}

void FusedQuantGemm::DestroyDownProjMmqLayout(const MmqWeightInfo &layout) {
  if (layout.data) (void)hipFree(const_cast<void *>(layout.data));
}

bool FusedQuantGemm::SupportsDownProjMmq(int quant_type) {
  return quant_type == static_cast<int>(TensorType::Q4_K) ||
         quant_type == static_cast<int>(TensorType::Q6_K);
}

int FusedQuantGemm::GetDownProjMmqThreshold(int quant_type, int m, int n, int k) {
  (void)m;
  (void)n;
  (void)k;
  (void)quant_type;
  const int override_m = NativeExecutionPolicy::FromEnv().downproj_mmq_min_batch_override;
  if (override_m >= 0) return override_m;
  return 3;
}

// ---- Producers fused into their consumer ----

namespace {

template <size_t C>
bool LaunchNormGroup(const std::array<PackedProjectionSpec, C> &p, const void *residual,
                     int residual_dtype, const uint16_t *norm_weight, float eps, int M, int K,
                     hipStream_t stream, const NativeExecutionPolicy *policy) {
  if (!residual || Resolve(policy).disable_fused_gemv) return false;
  const void *W[C];
  void *Y[C];
  int N[C];
  for (size_t i = 0; i < C; ++i) {
    if (!Usable(p[i].weight, residual, p[i].output)) return false;
    if (p[i].weight.quant_type != p[0].weight.quant_type) return false;
    if (!ViewCovers(p[i].weight, p[i].output_cols, K)) return false;
    W[i] = p[i].weight.data;
    Y[i] = p[i].output;
    N[i] = p[i].output_cols;
  }
  const FusedDispatchGeometry g{M, N[0], K, static_cast<int>(C), false, norm_weight != nullptr};
  if (!FusedQuantGemm::ShouldUseFusedPath(p[0].weight.quant_type, g)) return false;
  return ifx_qgemv_grouped_rmsnorm(p[0].weight.quant_type, static_cast<int>(C), W, Y, N, residual,
                                   residual_dtype, norm_weight, eps, IFX_OUT_F16, IFX_STORE, M, K,
                                   stream) == IFX_OK;
}

bool LaunchQuantizeAccum(const QuantizedWeightInfo &w, const void *input, int input_dtype,
                         float *output, int M, int N, int K, hipStream_t stream,
                         const NativeExecutionPolicy *policy) {
  if (!Usable(w, input, output) || Resolve(policy).disable_fused_gemv) return false;
  if (!ViewCovers(w, N, K)) return false;
  const void *W[1] = {w.data};
  void *Y[1] = {output};
  const int NN[1] = {N};
  return ifx_qgemv_grouped_rmsnorm(w.quant_type, 1, W, Y, NN, input, input_dtype, nullptr, 0.0f,
                                   IFX_OUT_F32, IFX_ACCUM, M, K, stream) == IFX_OK;
}

}  // namespace

bool FusedQuantGemm::FusedRmsNormGemvQ8_1Pair(const std::array<PackedProjectionSpec, 2> &projections,
                                              const float *residual, const uint16_t *norm_weight,
                                              int M, int K, float rms_norm_eps, hipStream_t stream,
                                              const NativeExecutionPolicy *policy) {
  if (!norm_weight) return false;
  return LaunchNormGroup(projections, residual, IFX_OUT_F32, norm_weight, rms_norm_eps, M, K,
                         stream, policy);
}

bool FusedQuantGemm::FusedRmsNormGemvQ8_1Triple(
    const std::array<PackedProjectionSpec, 3> &projections, const float *residual,
    const uint16_t *norm_weight, int M, int K, float rms_norm_eps, hipStream_t stream,
    const NativeExecutionPolicy *policy) {
  if (!norm_weight) return false;
  return LaunchNormGroup(projections, residual, IFX_OUT_F32, norm_weight, rms_norm_eps, M, K,
                         stream, policy);
}

bool FusedQuantGemm::QuantizeGemvQ8_1AccumF32(const QuantizedWeightInfo &weight,
                                              const float *input, float *output, int M, int N,
                                              int K, hipStream_t stream,
                                              const NativeExecutionPolicy *policy) {
  return LaunchQuantizeAccum(weight, input, IFX_OUT_F32, output, M, N, K, stream, policy);
}

bool FusedQuantGemm::QuantizeGemvQ8_1AccumF32(const QuantizedWeightInfo &weight,
                                              const uint16_t *input, float *output, int M, int N,
                                              int K, hipStream_t stream,
                                              const NativeExecutionPolicy *policy) {
  return LaunchQuantizeAccum(weight, input, IFX_OUT_F16, output, M, N, K, stream, policy);
}

bool FusedQuantGemm::FusedRmsNormGateUpSiluGemvQ8_1WithEpilogue(
    const QuantizedWeightInfo &gate_raw, const QuantizedWeightInfo &up_raw, const float *residual,
    const uint16_t *norm_weight, float rms_norm_eps, uint16_t *output, void *act_q8_1_out, int M,
    int N, int K, hipStream_t stream) {
  if (!Usable(gate_raw, residual, output) || !Usable(up_raw, residual, output) || !norm_weight)
    return false;
  if (gate_raw.quant_type != up_raw.quant_type) return false;
  if (!ViewCovers(gate_raw, N, K) || !ViewCovers(up_raw, N, K)) return false;
  return ifx_qgemv_gate_up_silu_rmsnorm(gate_raw.quant_type, gate_raw.data, up_raw.data, residual,
                                        IFX_OUT_F32, norm_weight, rms_norm_eps, output,
                                        IFX_OUT_F16, act_q8_1_out, M, N, K, stream) == IFX_OK;
}

int64_t FusedQuantGemm::ReductionWorkspaceBytes(int quant_type, int count, const int *N,
                                                bool f16_out, int M, int K) {
  return ifx_qgemv_workspace_bytes(quant_type, count, N, f16_out ? IFX_OUT_F16 : IFX_OUT_F32, M,
                                   K);
}

}  // namespace rocm
}  // namespace inferflux
