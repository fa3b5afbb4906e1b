// test_down_proj_mmq.cpp -- the down-projection MMQ and operator-selection
// half of the C++ FusedQuantGemm mirror (include/ifx_fused_quant_gemm.h,
// include/ifx_native_dispatch.h), in the manner of the reference's
// tests/unit/test_native_forward.cpp.
//
//   test_down_proj_mmq policy   host-only cases: the reference's operator-
//                               selection expectations
//                               (test_native_forward.cpp:6380-6660,
//                               6740-6960), each kept or marked where the
//                               MI355X thresholds differ, and argument
//                               rejection of the new entry points
//   test_down_proj_mmq gpu      BuildDownProjMmqLayout + DownProjMmq on the
//                               BASELINE down projections and the
//                               producer-fused extensions, against the oracle
#include "test_common.h"

#include "../../include/ifx_native_dispatch.h"

using inferflux::rocm::InferfluxCudaDispatchBucket;
using inferflux::rocm::InferfluxCudaDispatchPhase;
using inferflux::rocm::MmqWeightInfo;
using DownOp = inferflux::rocm::FusedQuantGemm::DownProjOperator;
using FfnOp = inferflux::rocm::FusedQuantGemm::FfnProjOperator;
namespace rocm = inferflux::rocm;

namespace {

DownOp Down(int qt, FusedDispatchGeometry g, bool q81, bool packed, bool mmq,
            const NativeExecutionPolicy *p = nullptr) {
  return FusedQuantGemm::SelectDownProjOperator(qt, g, q81, packed, mmq, p);
}

FfnOp Ffn(int qt, FusedDispatchGeometry g, bool q81, bool packed,
          const NativeExecutionPolicy *p = nullptr) {
  return FusedQuantGemm::SelectFfnProjOperator(qt, qt, g, q81, packed, p);
}

// ---------------------------------------------------------------- policy
void TestDownSelection() {
  std::printf("[down-proj selection]\n");
  EXPECT(FusedQuantGemm::SupportsDownProjMmq(Q4_K));
  EXPECT(FusedQuantGemm::SupportsDownProjMmq(Q6_K));
  EXPECT(!FusedQuantGemm::SupportsDownProjMmq(Q8_0));
  EXPECT(FusedQuantGemm::kDownProjMmqTileCols == 32);
  // invalid geometry (test_native_forward.cpp:6392-6402)
  EXPECT(Down(Q4_K, {0, 4096, 11008, 1, true, false}, true, true, true) == DownOp::kFallback);
  EXPECT(Down(Q4_K, {1, 0, 11008, 1, true, false}, true, true, true) == DownOp::kFallback);
  // small Q4_K decode stays on the Q8_1 GEMV (:6404-6413)
  EXPECT(Down(Q4_K, {1, 4096, 11008, 1, true, false}, true, true, true) == DownOp::kQ81Gemv);
  // the hot 2048 x 11008 geometry at M = 1 / 2, with and without the
  // experimental switches (:6415-6560)
  for (int qt : {Q4_K, Q6_K}) {
    EXPECT(Down(qt, {1, 2048, 11008, 1, true, false}, true, true, true) == DownOp::kQ81GemvHotFixed);
    EXPECT(Down(qt, {2, 2048, 11008, 1, true, false}, true, true, true) ==
           DownOp::kQ81GemvRowPairHotFixed);
    setenv("INFERFLUX_ENABLE_EXPERIMENTAL_Q8_1_DOWNPROJ_HOT_FIXED", "1", 1);
    setenv("INFERFLUX_ENABLE_EXPERIMENTAL_Q8_1_DOWNPROJ_ROWPAIR_HOT_FIXED", "1", 1);
    EXPECT(Down(qt, {1, 2048, 11008, 1, true, false}, true, true, true) == DownOp::kQ81GemvHotFixed);
    EXPECT(Down(qt, {2, 2048, 11008, 1, true, false}, true, true, true) ==
           DownOp::kQ81GemvRowPairHotFixed);
    unsetenv("INFERFLUX_ENABLE_EXPERIMENTAL_Q8_1_DOWNPROJ_HOT_FIXED");
    unsetenv("INFERFLUX_ENABLE_EXPERIMENTAL_Q8_1_DOWNPROJ_ROWPAIR_HOT_FIXED");
  }
  // four-row Q6_K decode (:6562-6571): the reference selects the row-quad
  // GEMV; on gfx950 the tiled copy wins from M = 3 (GetDownProjMmqThreshold),
  // so with MMQ allowed it is kMmq, and the row-quad rule still follows
  // when MMQ is not allowed.
  EXPECT(Down(Q6_K, {4, 2048, 11008, 1, true, false}, true, true, true) == DownOp::kMmq);
  EXPECT(Down(Q6_K, {4, 2048, 11008, 1, true, false}, true, true, false) == DownOp::kQ81GemvRowQuad);
  EXPECT(Down(Q6_K, {3, 2048, 11008, 1, true, false}, true, true, false) == DownOp::kQ81GemvRowPair);
  // packed when Q8_1 is off (:6573-6582)
  EXPECT(Down(Q4_K, {1, 2048, 11008, 1, true, false}, false, true, false) == DownOp::kPackedGemv);
  // large batches (:6584-6593, 6640-6649): the reference promotes M = 256
  // to its MMQ kernel; here the tiled kernels stop at kDownProjMmqMaxM = 32
  // and larger M runs the prefill GEMM on the raw rows (GemvQ8_1), so M = 256
  // is not kMmq, and M = 32 is.
  for (int qt : {Q4_K, Q6_K}) {
    EXPECT(Down(qt, {256, 4096, 11008, 1, true, false}, true, true, true) == DownOp::kQ81GemvRowQuad);
    EXPECT(Down(qt, {32, 4096, 11008, 1, true, false}, true, true, true) == DownOp::kMmq);
    EXPECT(Down(qt, {33, 4096, 11008, 1, true, false}, true, true, true) == DownOp::kQ81GemvRowQuad);
  }
  // the batch override (:6595-6638): 1 promotes M = 1; junk is ignored
  EXPECT(FusedQuantGemm::GetDownProjMmqThreshold(Q4_K, 1, 4096, 11008) == 3);
  setenv("INFERFLUX_DOWNPROJ_MMQ_MIN_BATCH", "1", 1);
  EXPECT(FusedQuantGemm::GetDownProjMmqThreshold(Q4_K, 1, 4096, 11008) == 1);
  EXPECT(Down(Q4_K, {1, 4096, 11008, 1, true, false}, true, true, true) == DownOp::kMmq);
  setenv("INFERFLUX_DOWNPROJ_MMQ_MIN_BATCH", "not_a_number", 1);
  EXPECT(Down(Q4_K, {1, 4096, 11008, 1, true, false}, true, true, true) == DownOp::kQ81Gemv);
  setenv("INFERFLUX_DOWNPROJ_MMQ_MIN_BATCH", "65", 1);  // outside 1..64
  EXPECT(FusedQuantGemm::GetDownProjMmqThreshold(Q4_K, 1, 4096, 11008) == 3);
  unsetenv("INFERFLUX_DOWNPROJ_MMQ_MIN_BATCH");
  // generic batch rows: row pair for M = 2..3, row quad from 4
  EXPECT(Down(Q4_K, {2, 4096, 11008, 1, true, false}, true, true, false) == DownOp::kQ81GemvRowPair);
  EXPECT(Down(Q8_0, {4, 4096, 11008, 1, true, false}, true, true, true) == DownOp::kQ81Gemv);
  EXPECT(Down(Q4_K, {1, 4096, 11008, 1, true, false}, false, false, true) == DownOp::kFallback);

  EXPECT(std::string(FusedQuantGemm::DownProjOperatorName(DownOp::kMmq)) == "mmq");
  EXPECT(std::string(FusedQuantGemm::DownProjOperatorName(DownOp::kQ81GemvRowPairHotFixed)) ==
         "q8_1_gemv_row_pair_hot_fixed");
  EXPECT(std::string(FusedQuantGemm::DownProjOperatorMetricName(DownOp::kQ81Gemv, Q6_K, 8, 0)) ==
         "q8_1_mmvq");
  EXPECT(std::string(FusedQuantGemm::DownProjOperatorMetricName(DownOp::kQ81Gemv, Q6_K, 9, 0)) ==
         "q8_1_mmq");
  EXPECT(std::string(FusedQuantGemm::DownProjOperatorMetricName(DownOp::kMmq, Q6_K, 9, 0)) == "mmq");
}

void TestFfnSelection() {
  std::printf("[ffn selection]\n");
  // the named hot geometries (test_native_forward.cpp:6740-6818)
  const FusedDispatchGeometry hot_m1{1, 11008, 2048, 2, true, false};
  const FusedDispatchGeometry hot_m2{2, 11008, 2048, 2, true, false};
  setenv("INFERFLUX_ENABLE_EXPERIMENTAL_Q8_1_GROUPED_HOT_Q4K", "0", 1);
  EXPECT(!FusedQuantGemm::ShouldUseSpecializedQ8_1GroupedFastPath(Q4_K, hot_m1));
  setenv("INFERFLUX_ENABLE_EXPERIMENTAL_Q8_1_GROUPED_HOT_Q4K", "1", 1);
  EXPECT(FusedQuantGemm::ShouldUseSpecializedQ8_1GroupedFastPath(Q4_K, hot_m1));
  EXPECT(!FusedQuantGemm::ShouldUseSpecializedQ8_1GroupedFastPath(Q4_K, hot_m2));
  unsetenv("INFERFLUX_ENABLE_EXPERIMENTAL_Q8_1_GROUPED_HOT_Q4K");
  EXPECT(!FusedQuantGemm::ShouldUseSpecializedQ8_1GroupedFastPath(Q4_K, {1, 2048, 2048, 2, true, false}));
  EXPECT(!FusedQuantGemm::ShouldUseSpecializedQ8_1GroupedFastPath(Q4_K, {3, 11008, 2048, 2, true, false}));
  EXPECT(!FusedQuantGemm::ShouldUseSpecializedQ8_1GroupedFastPath(Q4_K, {1, 11008, 4096, 2, true, false}));
  EXPECT(!FusedQuantGemm::ShouldUseSpecializedQ8_1GroupedFastPath(Q4_K, {1, 11008, 2048, 3, true, false}));
  EXPECT(!FusedQuantGemm::ShouldUseSpecializedQ8_1GroupedFastPath(Q6_K, hot_m1));
  NativeExecutionPolicy on, off;
  off.enable_experimental_q81_grouped_rowpair_w4 = false;
  EXPECT(FusedQuantGemm::ShouldUseSpecializedQ8_1GroupedRowPairW4Path(Q4_K, hot_m2, &on));
  EXPECT(!FusedQuantGemm::ShouldUseSpecializedQ8_1GroupedRowPairW4Path(Q4_K, hot_m2, &off));
  EXPECT(!FusedQuantGemm::ShouldUseSpecializedQ8_1GroupedRowPairW4Path(Q4_K, hot_m1, &on));
  EXPECT(!FusedQuantGemm::ShouldUseSpecializedQ8_1GroupedRowPairW4Path(Q4_K, {2, 2048, 2048, 2, true, false}, &on));
  EXPECT(!FusedQuantGemm::ShouldUseSpecializedQ8_1GroupedRowPairW4Path(Q4_K, {2, 11008, 4096, 2, true, false}, &on));
  EXPECT(!FusedQuantGemm::ShouldUseSpecializedQ8_1GroupedRowPairW4Path(Q4_K, {2, 11008, 2048, 3, true, false}, &on));
  EXPECT(!FusedQuantGemm::ShouldUseSpecializedQ8_1GroupedRowPairW4Path(Q6_K, hot_m2, &on));

  // the FFN ladder (:6820-6900), all as the reference
  NativeExecutionPolicy p;
  EXPECT(Ffn(Q4_K, {1, 11008, 2048, 2, true, true}, true, true, &p) == FfnOp::kQ81GroupHotQ4K);
  EXPECT(Ffn(Q4_K, {2, 11008, 2048, 2, true, true}, true, true, &p) == FfnOp::kQ81GroupRowPairW4);
  EXPECT(Ffn(Q4_K, {3, 11008, 2048, 2, true, true}, true, true, &p) == FfnOp::kQ81GroupMmq3);
  EXPECT(Ffn(Q4_K, {4, 11008, 2048, 2, true, true}, true, true, &p) == FfnOp::kQ81GroupMmq3);
  p.enable_experimental_q81_grouped_rowpair_w4 = false;
  EXPECT(Ffn(Q4_K, {2, 11008, 2048, 2, true, true}, true, true, &p) == FfnOp::kQ81Group);
  p.enable_experimental_q81_grouped_rowquad_m4 = true;
  EXPECT(Ffn(Q4_K, {4, 11008, 2048, 2, true, true}, true, true, &p) == FfnOp::kQ81GroupRowQuadM4);
  EXPECT(Ffn(Q4_K, {3, 11008, 2048, 2, true, true}, true, true, &p) == FfnOp::kQ81GroupMmq3);
  EXPECT(Ffn(Q6_K, {1, 11008, 2048, 2, true, true}, true, true) == FfnOp::kQ81Group);
  EXPECT(Ffn(Q4_K, {1, 11008, 2048, 2, true, true}, false, true) == FfnOp::kPackedGroup);
  EXPECT(Ffn(Q4_K, {1, 11008, 2048, 1, true, true}, true, true) == FfnOp::kFallback);
  EXPECT(Ffn(Q4_K, {1, 11008, 2048, 2, true, true}, false, false) == FfnOp::kFallback);
  // the 14B gate/up at M = 32: the generic Q8_1 group (Q6_K) / MMQ3 (Q4_K)
  EXPECT(Ffn(Q4_K, {32, 13824, 5120, 2, true, true}, true, true) == FfnOp::kQ81GroupMmq3);
  EXPECT(Ffn(Q6_K, {32, 13824, 5120, 2, true, true}, true, true) == FfnOp::kQ81Group);

  EXPECT(std::string(FusedQuantGemm::FfnProjOperatorName(FfnOp::kQ81GroupRowPairW4)) ==
         "q8_1_group_row_pair_w4");
  EXPECT(std::string(FusedQuantGemm::FfnProjOperatorName(FfnOp::kFallback)) == "fallback");
  EXPECT(std::string(FusedQuantGemm::FfnProjOperatorMetricName(FfnOp::kQ81Group, Q4_K, 8, 0)) ==
         "q8_1_group_mmvq");
  EXPECT(std::string(FusedQuantGemm::FfnProjOperatorMetricName(FfnOp::kQ81Group, Q4_K, 9, 0)) ==
         "q8_1_group_mmq");
  EXPECT(std::string(FusedQuantGemm::FfnProjOperatorMetricName(FfnOp::kQ81Group, Q8_0, 9, 0)) ==
         "q8_1_group");
}

void TestRegistry() {
  std::printf("[registry]\n");
  EXPECT(rocm::BucketBatchRows(0) == InferfluxCudaDispatchBucket::k1);
  EXPECT(rocm::BucketBatchRows(2) == InferfluxCudaDispatchBucket::k2);
  EXPECT(rocm::BucketBatchRows(4) == InferfluxCudaDispatchBucket::k3_4);
  EXPECT(rocm::BucketBatchRows(5) == InferfluxCudaDispatchBucket::k5_8);
  EXPECT(rocm::BucketBatchRows(16) == InferfluxCudaDispatchBucket::k9_16);
  EXPECT(rocm::BucketBatchRows(17) == InferfluxCudaDispatchBucket::k17Plus);
  EXPECT(std::string(rocm::InferfluxCudaDispatchBucketName(InferfluxCudaDispatchBucket::k17Plus)) ==
         "17_plus");
  EXPECT(rocm::ParseInferfluxCudaDispatchPhase("prefill") == InferfluxCudaDispatchPhase::kPrefill);
  EXPECT(rocm::ParseInferfluxCudaDispatchPhase("x") == InferfluxCudaDispatchPhase::kUnknown);
  const auto prof = rocm::BuildInferfluxCudaDownProjDispatchProfile(
      InferfluxCudaDispatchPhase::kDecode, Q6_K, {8, 2048, 11008, 1, true, false}, true, false, true);
  const auto dec = rocm::SelectInferfluxCudaDownProjDispatchDecision(prof, NativeExecutionPolicy{});
  EXPECT(dec.op == DownOp::kMmq && std::string(dec.reason) == "mmq");
  EXPECT(rocm::DescribeInferfluxCudaDownProjDispatchDecision(prof, dec.reason) ==
         "phase=decode, quant=q6_k, q81_ready=true, packed_ready=false, mmq_ready=true, "
         "m_bucket=5_8, n_bucket=17_plus, k_bucket=17_plus, rule=mmq");

  // the policy wrappers (test_native_forward.cpp:6880-6960)
  NativeExecutionPolicy policy;
  const QuantizedWeightInfo raw{reinterpret_cast<const void *>(0x1), Q4_K, 2048LL * 11008LL};
  const MmqWeightInfo mmq{reinterpret_cast<const void *>(0x2), Q4_K, 2048, 11008,
                          FusedQuantGemm::kDownProjMmqTileCols};
  EXPECT(rocm::SelectInferfluxCudaDownProjOperator(raw, mmq, InferfluxCudaDispatchPhase::kDecode,
                                                   {1, 2048, 11008, 1, true, false}, false,
                                                   policy) == DownOp::kFallback);
  policy.disable_q81_activations = true;
  EXPECT(rocm::SelectInferfluxCudaDownProjOperator(raw, mmq, InferfluxCudaDispatchPhase::kDecode,
                                                   {1, 2048, 11008, 1, true, false}, true,
                                                   policy) == DownOp::kPackedGemv);
  policy.disable_q81_activations = false;
  // the MMQ operator needs a built layout and the policy switch
  EXPECT(rocm::SelectInferfluxCudaDownProjOperator(raw, mmq, InferfluxCudaDispatchPhase::kDecode,
                                                   {8, 2048, 11008, 1, true, false}, true,
                                                   policy) == DownOp::kMmq);
  EXPECT(rocm::SelectInferfluxCudaDownProjOperator(raw, MmqWeightInfo{},
                                                   InferfluxCudaDispatchPhase::kDecode,
                                                   {8, 2048, 11008, 1, true, false}, true,
                                                   policy) == DownOp::kQ81GemvRowQuad);
  policy.enable_downproj_mmq = false;
  EXPECT(rocm::SelectInferfluxCudaDownProjOperator(raw, mmq, InferfluxCudaDispatchPhase::kDecode,
                                                   {8, 2048, 11008, 1, true, false}, true,
                                                   policy) == DownOp::kQ81GemvRowQuad);
  policy.enable_downproj_mmq = true;
  policy.force_cublas = true;
  const QuantizedWeightInfo graw{reinterpret_cast<const void *>(0x1), Q4_K, 2048LL * 11008LL};
  EXPECT(rocm::SelectInferfluxCudaFfnProjOperator(graw, graw, InferfluxCudaDispatchPhase::kDecode,
                                                  {1, 11008, 2048, 2, true, true}, true,
                                                  policy) == FfnOp::kFallback);
  policy.force_cublas = false;
  EXPECT(rocm::SelectInferfluxCudaFfnProjOperator(graw, graw, InferfluxCudaDispatchPhase::kDecode,
                                                  {1, 11008, 2048, 2, true, true}, true,
                                                  policy) == FfnOp::kQ81GroupHotQ4K);
  EXPECT(rocm::SelectInferfluxCudaFfnProjOperator(graw, graw, InferfluxCudaDispatchPhase::kPrefill,
                                                  {1, 11008, 2048, 2, true, true}, true,
                                                  policy) == FfnOp::kQ81Group);
  EXPECT(rocm::SelectInferfluxCudaFfnProjOperator(graw, graw, InferfluxCudaDispatchPhase::kDecode,
                                                  {3, 11008, 2048, 2, true, true}, true,
                                                  policy) == FfnOp::kQ81GroupMmq3);
  policy.enable_experimental_q81_grouped_rowquad_m4 = true;
  EXPECT(rocm::SelectInferfluxCudaFfnProjOperator(graw, graw, InferfluxCudaDispatchPhase::kDecode,
                                                  {4, 11008, 2048, 2, true, true}, true,
                                                  policy) == FfnOp::kQ81GroupRowQuadM4);
  EXPECT(rocm::ProjectionQuantLabel(raw) == "q4_k");
  EXPECT(rocm::ProjectionGroupQuantLabel(raw, QuantizedWeightInfo{raw.data, Q6_K, 1}) == "mixed");
  EXPECT(rocm::ProjectionHasGraphSafeKernel(raw, {8, 11008, 2048, 1, true, true}, true,
                                            NativeExecutionPolicy{}));
  EXPECT(!rocm::ProjectionHasGraphSafeKernel(raw, {8, 11008, 2048, 1, true, true}, false,
                                             NativeExecutionPolicy{}));
}

// The entry points reject bad calls before launching anything.
void TestRejects() {
  std::printf("[down-proj rejects]\n");
  const uint8_t dummy[64] = {};
  uint16_t out[4];
  MmqWeightInfo l{dummy, Q6_K, 2048, 11008, FusedQuantGemm::kDownProjMmqTileCols};
  EXPECT(!FusedQuantGemm::DownProjMmq(l, dummy, out, 1, 2048, 10752, nullptr));  // K != cols
  EXPECT(!FusedQuantGemm::DownProjMmq(l, dummy, out, 1, 2047, 11008, nullptr));  // N != rows
  EXPECT(!FusedQuantGemm::DownProjMmq(l, dummy, out, 33, 2048, 11008, nullptr));
  EXPECT(!FusedQuantGemm::DownProjMmq(l, nullptr, out, 1, 2048, 11008, nullptr));
  MmqWeightInfo ref_tile = l;
  ref_tile.tile_cols = 8;  // the reference's CUDA layout is not this one
  EXPECT(!FusedQuantGemm::DownProjMmq(ref_tile, dummy, out, 1, 2048, 11008, nullptr));
  MmqWeightInfo q8 = l;
  q8.quant_type = Q8_0;
  EXPECT(!FusedQuantGemm::DownProjMmq(q8, dummy, out, 1, 2048, 11008, nullptr));
  NativeExecutionPolicy off;
  off.enable_downproj_mmq = false;
  EXPECT(!FusedQuantGemm::DownProjMmq(l, dummy, out, 1, 2048, 11008, nullptr, &off));
  EXPECT(!FusedQuantGemm::IsDownProjMmqEnabled(&off));
  EXPECT(FusedQuantGemm::IsDownProjMmqEnabled());
  setenv("INFERFLUX_ENABLE_DOWNPROJ_MMQ", "0", 1);
  EXPECT(!FusedQuantGemm::IsDownProjMmqEnabled());
  EXPECT(!FusedQuantGemm::DownProjMmq(l, dummy, out, 1, 2048, 11008, nullptr));
  unsetenv("INFERFLUX_ENABLE_DOWNPROJ_MMQ");
  MmqWeightInfo built;
  EXPECT(!FusedQuantGemm::BuildDownProjMmqLayout(QuantizedWeightInfo{}, 16, 256, &built, nullptr));
  EXPECT(!FusedQuantGemm::BuildDownProjMmqLayout(QuantizedWeightInfo{dummy, Q4_K, 4096}, 16, 100,
                                                 &built, nullptr));
  EXPECT(!FusedQuantGemm::BuildDownProjMmqLayout(QuantizedWeightInfo{dummy, Q8_0, 4096}, 16, 256,
                                                 &built, nullptr));
  EXPECT(!FusedQuantGemm::BuildDownProjMmqLayout(QuantizedWeightInfo{dummy, Q4_K, 4095}, 16, 256,
                                                 &built, nullptr));  // view smaller than 16 x 256
  FusedQuantGemm::DestroyDownProjMmqLayout(MmqWeightInfo{});  // no-op
  // the fused producers: outside their kernels' range they are not handled
  std::array<PackedProjectionSpec, 2> pr{
      PackedProjectionSpec{QuantizedWeightInfo{dummy, Q6_K, 1 << 20}, out, 64},
      PackedProjectionSpec{QuantizedWeightInfo{dummy, Q6_K, 1 << 20}, out, 64}};
  const float *res = reinterpret_cast<const float *>(dummy);
  const uint16_t *nw = reinterpret_cast<const uint16_t *>(dummy);
  EXPECT(!FusedQuantGemm::FusedRmsNormGemvQ8_1Pair(pr, res, nw, 1, 2048, 1e-6f, nullptr));  // Q6_K
  pr[0].weight.quant_type = pr[1].weight.quant_type = Q4_K;
  EXPECT(!FusedQuantGemm::FusedRmsNormGemvQ8_1Pair(pr, res, nw, 3, 2048, 1e-6f, nullptr));  // M = 3
  EXPECT(!FusedQuantGemm::FusedRmsNormGemvQ8_1Pair(pr, res, nullptr, 1, 2048, 1e-6f, nullptr));
  EXPECT(!FusedQuantGemm::FusedRmsNormGateUpSiluGemvQ8_1WithEpilogue(
      pr[0].weight, pr[1].weight, res, nw, 1e-6f, out, nullptr, 1, 64, 4096, nullptr));  // K
}

// ------------------------------------------------------------------- gpu
// BuildDownProjMmqLayout + DownProjMmq (fp16), DownProjMmqF32 and
// DownProjMmqAccumF32 against the oracle; with a reduction workspace in the
// policy, two accumulate calls from the same base give the same bits.
void TestDownProj(int qtype, int M, int N, int K) {
  std::printf("[gpu down-proj mmq] qtype=%d M=%d N=%d K=%d\n", qtype, M, N, K);
  std::fflush(stdout);
  Problem p = MakeProblem(qtype, M, N, K, 31 * qtype + M + N);
  Dev dw(p.w.size()), da(p.a.size()), dy(static_cast<size_t>(M) * N * 4),
      dh(static_cast<size_t>(M) * N * 2);
  HIP_OK(hipMemcpy(dw.p, p.w.data(), p.w.size(), hipMemcpyHostToDevice));
  HIP_OK(hipMemcpy(da.p, p.a.data(), p.a.size(), hipMemcpyHostToDevice));
  hipStream_t s;
  HIP_OK(hipStreamCreate(&s));
  MmqWeightInfo layout;
  EXPECT(FusedQuantGemm::BuildDownProjMmqLayout(QuantizedWeightInfo{dw.p, qtype, int64_t{N} * K},
                                                N, K, &layout, s));
  EXPECT(layout.data && layout.rows == N && layout.cols == K && layout.quant_type == qtype &&
         layout.tile_cols == FusedQuantGemm::kDownProjMmqTileCols);
  if (!layout.data) return;
  // the selector sends this call to DownProjMmq from M = 3 on
  EXPECT((Down(qtype, {M, N, K, 1, true, false}, true, true, true) == DownOp::kMmq) == (M >= 3));

  std::vector<uint16_t> h(static_cast<size_t>(M) * N);
  EXPECT(FusedQuantGemm::DownProjMmq(layout, da.p, dh.as<uint16_t>(), M, N, K, s));
  HIP_OK(hipStreamSynchronize(s));
  HIP_OK(hipMemcpy(h.data(), dh.p, h.size() * 2, hipMemcpyDeviceToHost));
  EXPECT(RowsClose(HalfToFloat(h), p.ye, M, N, 1e-3, true));

  std::vector<float> y(static_cast<size_t>(M) * N);
  EXPECT(FusedQuantGemm::DownProjMmqF32(layout, da.p, dy.as<float>(), M, N, K, s));
  HIP_OK(hipStreamSynchronize(s));
  HIP_OK(hipMemcpy(y.data(), dy.p, y.size() * 4, hipMemcpyDeviceToHost));
  EXPECT(RowsClose(y, p.ye, M, N, 1e-3, false));

  // accumulate into a residual of 0.5: fp32 atomics (plain), then twice
  // with deterministic_reductions (the layout's workspace): the same bits
  const std::vector<float> base(y.size(), 0.5f);
  NativeExecutionPolicy ordered;
  ordered.deterministic_reductions = true;
  std::vector<float> first;
  for (int pass = 0; pass < 3; ++pass) {
    HIP_OK(hipMemcpy(dy.p, base.data(), base.size() * 4, hipMemcpyHostToDevice));
    EXPECT(FusedQuantGemm::DownProjMmqAccumF32(layout, da.p, dy.as<float>(), M, N, K, s,
                                               pass == 0 ? nullptr : &ordered));
    HIP_OK(hipStreamSynchronize(s));
    HIP_OK(hipMemcpy(y.data(), dy.p, y.size() * 4, hipMemcpyDeviceToHost));
    std::vector<float> d(y);
    for (auto &v : d) v -= 0.5f;
    EXPECT(RowsClose(d, p.ye, M, N, 1e-3, false));
    if (pass == 1) first = y;
    if (pass == 2) EXPECT(std::memcmp(first.data(), y.data(), y.size() * 4) == 0);
  }
  // fp16 accumulate (the reference's half residual): ordered, twice
  std::vector<uint16_t> hbase(h.size(), orc_f32_to_f16(0.5f)), h1;
  for (int pass = 0; pass < 2; ++pass) {
    HIP_OK(hipMemcpy(dh.p, hbase.data(), hbase.size() * 2, hipMemcpyHostToDevice));
    EXPECT(FusedQuantGemm::DownProjMmq(layout, da.p, dh.as<uint16_t>(), M, N, K, s));
    HIP_OK(hipStreamSynchronize(s));
    HIP_OK(hipMemcpy(h.data(), dh.p, h.size() * 2, hipMemcpyDeviceToHost));
    if (pass == 0) h1 = h;
    else EXPECT(h == h1);
  }
  FusedQuantGemm::DestroyDownProjMmqLayout(layout);
  HIP_OK(hipStreamDestroy(s));
}

// deterministic_reductions on the raw-weight entries: a launch that splits
// K needs reduction_workspace (else it is not handled); with it, two calls
// give the same bits and pass the oracle bar.  Without the flag a large
// enough workspace gives the same ordered reduction, a smaller one the
// atomic form.
void TestDeterministicGemv(int qtype, int M, int N, int K) {
  std::printf("[gpu deterministic gemv] qtype=%d M=%d N=%d K=%d\n", qtype, M, N, K);
  std::fflush(stdout);
  Problem p = MakeProblem(qtype, M, N, K, 77 * qtype + M);
  Dev dw(p.w.size()), da(p.a.size()), dy(static_cast<size_t>(M) * N * 4);
  HIP_OK(hipMemcpy(dw.p, p.w.data(), p.w.size(), hipMemcpyHostToDevice));
  HIP_OK(hipMemcpy(da.p, p.a.data(), p.a.size(), hipMemcpyHostToDevice));
  const QuantizedWeightInfo w{dw.p, qtype, int64_t{N} * K};
  const int NN[1] = {N};
  const int64_t wsb = FusedQuantGemm::ReductionWorkspaceBytes(qtype, 1, NN, false, M, K);
  NativeExecutionPolicy det;
  det.deterministic_reductions = true;
  float *y = dy.as<float>();
  if (wsb > 0) EXPECT(!FusedQuantGemm::GemvQ8_1F32(w, da.p, y, M, N, K, nullptr, &det));
  Dev ws(static_cast<size_t>(wsb) + 256);
  HIP_OK(hipMemset(ws.p, 0, static_cast<size_t>(wsb) + 256));
  det.reduction_workspace = ws.p;
  det.reduction_workspace_bytes = wsb;
  std::vector<float> a(static_cast<size_t>(M) * N), b(a.size());
  EXPECT(FusedQuantGemm::GemvQ8_1F32(w, da.p, y, M, N, K, nullptr, &det));
  HIP_OK(hipDeviceSynchronize());
  HIP_OK(hipMemcpy(a.data(), y, a.size() * 4, hipMemcpyDeviceToHost));
  EXPECT(FusedQuantGemm::GemvQ8_1F32(w, da.p, y, M, N, K, nullptr, &det));
  HIP_OK(hipDeviceSynchronize());
  HIP_OK(hipMemcpy(b.data(), y, b.size() * 4, hipMemcpyDeviceToHost));
  EXPECT(a == b);
  EXPECT(RowsClose(a, p.ye, M, N, 1e-3, false));
  // without the flag, the caller's workspace alone selects the ordered
  // reduction: the same bits again
  NativeExecutionPolicy scratch;
  scratch.reduction_workspace = ws.p;
  scratch.reduction_workspace_bytes = wsb;
  EXPECT(FusedQuantGemm::GemvQ8_1F32(w, da.p, y, M, N, K, nullptr, &scratch));
  HIP_OK(hipDeviceSynchronize());
  HIP_OK(hipMemcpy(b.data(), y, b.size() * 4, hipMemcpyDeviceToHost));
  EXPECT(a == b);
  // a workspace below the launch's size without the flag: the atomic form
  // still runs (and passes the bar)
  if (wsb > 0) {
    scratch.reduction_workspace_bytes = wsb - 256;
    EXPECT(FusedQuantGemm::GemvQ8_1F32(w, da.p, y, M, N, K, nullptr, &scratch));
    HIP_OK(hipDeviceSynchronize());
    HIP_OK(hipMemcpy(b.data(), y, b.size() * 4, hipMemcpyDeviceToHost));
    EXPECT(RowsClose(b, p.ye, M, N, 1e-3, false));
  }
  if (wsb == 0) {
    // accumulate into a fixed base: with the flag and no workspace, the
    // same bits on every call; without a policy (the plain entry, whose
    // fp32 accumulate launches at 9 <= M <= 16 split K with atomics) within
    // the bar
    std::vector<float> base(a.size());
    std::vector<double> yb(p.ye);
    for (size_t i = 0; i < base.size(); ++i) {
      base[i] = 0.25f * static_cast<float>(i % 7) - 0.5f;
      yb[i] += base[i];
    }
    auto run = [&](const NativeExecutionPolicy *pol, std::vector<float> &out) {
      HIP_OK(hipMemcpy(y, base.data(), base.size() * 4, hipMemcpyHostToDevice));
      EXPECT(FusedQuantGemm::GemvQ8_1AccumF32(w, da.p, y, M, N, K, nullptr, pol));
      HIP_OK(hipDeviceSynchronize());
      HIP_OK(hipMemcpy(out.data(), y, out.size() * 4, hipMemcpyDeviceToHost));
    };
    NativeExecutionPolicy det0;
    det0.deterministic_reductions = true;
    run(&det0, a);
    run(&det0, b);
    EXPECT(a == b);
    EXPECT(RowsClose(a, yb, M, N, 1e-3, false));
    run(nullptr, b);
    EXPECT(RowsClose(b, yb, M, N, 1e-3, false));
  }
}

// The producer-fused extensions against the oracle chain: RMSNorm + Q8_1
// (orc_rmsnorm_quantize_q8_1) then the exact GEMV.
void TestFusedProducers() {
  std::printf("[gpu fused producers]\n");
  std::fflush(stdout);
  const int M = 1, K = 2048;
  const std::array<int, 3> Ns = {2048, 256, 256};
  Rng r(91);
  std::vector<float> x(static_cast<size_t>(M) * K);
  std::vector<uint16_t> nw(K);
  for (auto &v : x) v = r.normal();
  // small norm weights keep h = silu(g) * u inside the fp16 range
  for (auto &v : nw) v = orc_f32_to_f16(0.01f + 0.01f * r.uniform());
  std::vector<uint8_t> a(static_cast<size_t>(M) * (K / 32) * 36);
  orc_rmsnorm_quantize_q8_1(x.data(), nw.data(), a.data(), M, K, 1e-6f);
  Dev dx(x.size() * 4), dnw(K * 2);
  HIP_OK(hipMemcpy(dx.p, x.data(), x.size() * 4, hipMemcpyHostToDevice));
  HIP_OK(hipMemcpy(dnw.p, nw.data(), K * 2, hipMemcpyHostToDevice));
  std::vector<std::vector<uint8_t>> ws;
  std::vector<std::unique_ptr<Dev>> dws, dys;
  std::array<PackedProjectionSpec, 3> spec{};
  for (size_t i = 0; i < 3; ++i) {
    ws.push_back(MakeBlocks(Q4_K, Ns[i], K, 500 + i));
    dws.emplace_back(new Dev(ws[i].size()));
    dys.emplace_back(new Dev(static_cast<size_t>(M) * Ns[i] * 4));
    HIP_OK(hipMemcpy(dws[i]->p, ws[i].data(), ws[i].size(), hipMemcpyHostToDevice));
    spec[i] = PackedProjectionSpec{QuantizedWeightInfo{dws[i]->p, Q4_K, int64_t{Ns[i]} * K},
                                   dys[i]->as<uint16_t>(), Ns[i]};
  }
  EXPECT(FusedQuantGemm::FusedRmsNormGemvQ8_1Triple(spec, dx.as<float>(), dnw.as<uint16_t>(), M, K,
                                                    1e-6f, nullptr));
  HIP_OK(hipDeviceSynchronize());
  for (size_t i = 0; i < 3; ++i) {
    std::vector<double> ye(static_cast<size_t>(M) * Ns[i]);
    orc_gemv_exact(Q4_K, ws[i].data(), a.data(), ye.data(), M, Ns[i], K, 8);
    std::vector<uint16_t> h(ye.size());
    HIP_OK(hipMemcpy(h.data(), dys[i]->p, h.size() * 2, hipMemcpyDeviceToHost));
    EXPECT(RowsClose(HalfToFloat(h), ye, M, Ns[i], 1e-3, true));
  }
  const std::array<PackedProjectionSpec, 2> pair{spec[1], spec[2]};
  EXPECT(FusedQuantGemm::FusedRmsNormGemvQ8_1Pair(pair, dx.as<float>(), dnw.as<uint16_t>(), M, K,
                                                  1e-6f, nullptr));
  HIP_OK(hipDeviceSynchronize());
  // the O projection: Q8_1(x) then += into an fp32 residual of 0.25
  std::vector<uint8_t> aq(a.size());
  orc_quantize_q8_1_f32(x.data(), aq.data(), M, K);
  std::vector<double> ye(static_cast<size_t>(M) * Ns[0]);
  orc_gemv_exact(Q4_K, ws[0].data(), aq.data(), ye.data(), M, Ns[0], K, 8);
  Dev dres(static_cast<size_t>(M) * Ns[0] * 4);
  std::vector<float> y(static_cast<size_t>(M) * Ns[0], 0.25f);
  HIP_OK(hipMemcpy(dres.p, y.data(), y.size() * 4, hipMemcpyHostToDevice));
  EXPECT(FusedQuantGemm::QuantizeGemvQ8_1AccumF32(spec[0].weight, dx.as<float>(), dres.as<float>(),
                                                  M, Ns[0], K, nullptr));
  HIP_OK(hipDeviceSynchronize());
  HIP_OK(hipMemcpy(y.data(), dres.p, y.size() * 4, hipMemcpyDeviceToHost));
  for (auto &v : y) v -= 0.25f;
  EXPECT(RowsClose(y, ye, M, Ns[0], 1e-3, false));
  // gate/up + SiLU with the RMSNorm producer fused in: h against
  // silu(g) * u of the oracle's exact g and u, within the bar the GEMV bar
  // carries through the product (|dh| <= |silu'(g) u| eg + |silu(g)| eu)
  const int N = 256;
  Dev dh(static_cast<size_t>(M) * N * 2), dq(static_cast<size_t>(M) * (N / 32) * 36);
  EXPECT(FusedQuantGemm::FusedRmsNormGateUpSiluGemvQ8_1WithEpilogue(
      spec[1].weight, spec[2].weight, dx.as<float>(), dnw.as<uint16_t>(), 1e-6f,
      dh.as<uint16_t>(), dq.p, M, N, K, nullptr));
  HIP_OK(hipDeviceSynchronize());
  std::vector<double> g(N), u(N);
  orc_gemv_exact(Q4_K, ws[1].data(), a.data(), g.data(), M, N, K, 8);
  orc_gemv_exact(Q4_K, ws[2].data(), a.data(), u.data(), M, N, K, 8);
  double ng = 0, nu = 0;
  for (int n = 0; n < N; ++n) ng += g[n] * g[n], nu += u[n] * u[n];
  const double eg = 1e-3 * std::sqrt(ng), eu = 1e-3 * std::sqrt(nu);
  std::vector<uint16_t> hh(N);
  HIP_OK(hipMemcpy(hh.data(), dh.p, N * 2, hipMemcpyDeviceToHost));
  for (int n = 0; n < N; ++n) {
    const double sg = 1.0 / (1.0 + std::exp(-g[n])), silu = g[n] * sg;
    const double dsilu = sg * (1.0 + g[n] * (1.0 - sg));
    const double he = silu * u[n];
    const double lim = std::fabs(dsilu * u[n]) * eg + std::fabs(silu) * eu + std::fabs(he) / 1024;
    if (!(std::fabs(orc_f16_to_f32(hh[n]) - he) <= lim)) {
      std::printf("  h[%d] = %g, expected %g (bar %g)\n", n, orc_f16_to_f32(hh[n]), he, lim);
      ++g_failures;
      break;
    }
  }
}

}  // namespace

int main(int argc, char **argv) {
  const std::string mode = argc > 1 ? argv[1] : "policy";
  if (mode == "policy") {
    TestDownSelection();
    TestFfnSelection();
    TestRegistry();
    TestRejects();
  } else if (mode == "gpu") {
    TestDownProj(Q4_K, 4, 16, 256);  // the reference's own case (test_native_forward.cpp:4861)
    TestDownProj(Q6_K, 1, 2048, 11008);  // 3B down projection
    TestDownProj(Q6_K, 2, 2048, 11008);
    TestDownProj(Q6_K, 4, 2048, 11008);
    TestDownProj(Q6_K, 8, 2048, 11008);
    TestDownProj(Q6_K, 16, 5120, 13824);  // 14B down projection
    TestDownProj(Q6_K, 32, 5120, 13824);
    TestDownProj(Q4_K, 1, 2048, 11008);
    TestDownProj(Q4_K, 8, 2048, 11008);
    TestDownProj(Q4_K, 32, 1000, 2048);  // a partial last tile
    TestDeterministicGemv(Q6_K, 8, 2048, 11008);  // slot GEMV, K split
    TestDeterministicGemv(Q4_K, 32, 5120, 5120);  // fp16-dequant GEMV, K split
    TestDeterministicGemv(Q4_K, 1, 2048, 2048);   // no split
    TestDeterministicGemv(Q4_K, 16, 5120, 5120);  // accumulate: MMVQ, or the atomic split
    TestFusedProducers();
  } else {
    std::printf("usage: %s policy|gpu\n", argv[0]);
    return 2;
  }
  std::printf("%s: %d failure(s)\n", mode.c_str(), g_failures);
  return g_failures ? 1 : 0;
}
