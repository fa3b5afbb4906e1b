// test_fused_quant_gemm.cpp -- tests of the C++ FusedQuantGemm mirror
// (include/ifx_fused_quant_gemm.h), in the manner of the reference's
// tests/unit/test_native_forward.cpp: the policy cases (thresholds,
// argument rejection, the disable switch) run without a GPU; the GPU cases
// run each entry point on seeded blocks and compare with the CPU oracle
// (oracle/ifx_oracle.c, linked as the checker).
//
//   test_fused_quant_gemm policy   host-only cases
//   test_fused_quant_gemm gpu      device cases (needs a GPU)
#include "test_common.h"

namespace {

// ---------------------------------------------------------------- policy
void TestPolicy() {
  std::printf("[policy]\n");
  EXPECT(FusedQuantGemm::SupportsQ8_1Activations(Q4_K));
  EXPECT(FusedQuantGemm::SupportsQ8_1Activations(Q6_K));
  EXPECT(FusedQuantGemm::SupportsQ8_1Activations(Q8_0));
  EXPECT(!FusedQuantGemm::SupportsQ8_1Activations(Q8_1));
  EXPECT(!FusedQuantGemm::SupportsQ8_1Activations(0));
  EXPECT(FusedQuantGemm::SupportsQ8_1Activations(15));  // Q8_K, as the reference
  EXPECT(FusedQuantGemm::SupportsQ8_1Activations(13));  // Q5_K (no reference kernel)
  EXPECT(!FusedQuantGemm::SupportsQ8_1Activations(16));
  // Q5_K / Q8_K: GEMV only, M <= 64 (the reference's Q8_K limit)
  EXPECT(FusedQuantGemm::GetAdaptiveThreshold(15) == 64);
  EXPECT(FusedQuantGemm::ShouldUseFusedPath(15, 64));
  EXPECT(!FusedQuantGemm::ShouldUseFusedPath(15, 65));
  EXPECT(!FusedQuantGemm::ShouldUseFusedPath(13, 512));
  EXPECT(FusedQuantGemm::SelectKernel(13, 32, 4096, 4096) == KernelFamily::kGemv);
  EXPECT(FusedQuantGemm::SelectKernel(15, 64, 4096, 4096) == KernelFamily::kGemv);
  EXPECT(FusedQuantGemm::SelectKernel(15, 65, 4096, 4096) == KernelFamily::kNone);

  // thresholds: no crossover to a fallback on gfx950
  EXPECT(FusedQuantGemm::GetAdaptiveThreshold(Q4_K) == FusedQuantGemm::kMaxFusedM);
  {  // the geometry narrows it: fused RMSNorm (Q4_K, M <= 2, activation rows in
     // 64 KiB of LDS) and 32-bit activation offsets
    FusedDispatchGeometry g{1, 2048, 2048, 1, false, true};
    EXPECT(FusedQuantGemm::GetGeometryAwareThreshold(Q4_K, g) == 2);
    EXPECT(FusedQuantGemm::GetGeometryAwareThreshold(Q6_K, g) == 0);
    EXPECT(!FusedQuantGemm::ShouldUseFusedPath(Q4_K, FusedDispatchGeometry{3, 2048, 2048, 1, false, true}));
    g.K = 40960;  // an LDS row of 56320 bytes: one row in 64 KiB
    EXPECT(FusedQuantGemm::GetGeometryAwareThreshold(Q4_K, g) == 1);
    FusedDispatchGeometry h{1, 64, 2048, 1, false, false};
    EXPECT(FusedQuantGemm::GetGeometryAwareThreshold(Q4_K, h) == 1864135);  // (2^32 - 1) / 2304
    h.K = 1 << 26;  // 2^21 blocks of 36 bytes per row
    EXPECT(FusedQuantGemm::GetGeometryAwareThreshold(Q4_K, h) == 56);
  }
  EXPECT(FusedQuantGemm::GetAdaptiveThreshold(1) == 0);
  EXPECT(!FusedQuantGemm::ShouldUseFusedPath(Q4_K, 0));
  EXPECT(FusedQuantGemm::ShouldUseFusedPath(Q4_K, 1));
  EXPECT(FusedQuantGemm::ShouldUseFusedPath(Q6_K, 64));
  EXPECT(FusedQuantGemm::ShouldUseFusedPath(Q8_0, 512));
  EXPECT(!FusedQuantGemm::ShouldUseFusedPath(Q8_1, 1));
  {
    FusedDispatchGeometry g{8, 4096, 2048, 4, true, false};
    EXPECT(!FusedQuantGemm::ShouldUseFusedPath(Q4_K, g));  // no 4-way group
    g.grouped_outputs = 3;
    EXPECT(FusedQuantGemm::ShouldUseFusedPath(Q4_K, g));
    g.K = 2080;  // not a whole number of Q4_K super-blocks
    EXPECT(!FusedQuantGemm::ShouldUseFusedPath(Q4_K, g));
    EXPECT(FusedQuantGemm::ShouldUseFusedPath(Q8_0, g));  // 65 Q8_0 blocks
  }
  EXPECT(FusedQuantGemm::SelectKernel(Q4_K, 1, 11008, 2048) == KernelFamily::kGemv);
  EXPECT(FusedQuantGemm::SelectKernel(Q4_K, 2, 11008, 2048) == KernelFamily::kGemv);
  EXPECT(FusedQuantGemm::SelectKernel(Q4_K, 8, 11008, 2048) == KernelFamily::kSkinnyMfma);
  EXPECT(FusedQuantGemm::SelectKernel(Q4_K, 3, 11008, 2048) == KernelFamily::kGemv);  // LDS-A GEMV
  EXPECT(FusedQuantGemm::SelectKernel(Q4_K, 4, 22016, 2048) == KernelFamily::kGemv);
  EXPECT(FusedQuantGemm::SelectKernel(Q4_K, 4, 11008, 2048) == KernelFamily::kSkinnyMfma);
  EXPECT(FusedQuantGemm::SelectKernel(Q6_K, 3, 11008, 2048) == KernelFamily::kSkinnyMfma);
  EXPECT(FusedQuantGemm::SelectKernel(Q6_K, 32, 5120, 13824) == KernelFamily::kF16DequantGemv);
  EXPECT(FusedQuantGemm::SelectKernel(Q6_K, 16, 5120, 13824) == KernelFamily::kSkinnyMfma);
  EXPECT(FusedQuantGemm::SelectKernel(Q4_K, 512, 27648, 5120) == KernelFamily::kF16DequantMfma);
  EXPECT(FusedQuantGemm::SelectKernel(Q4_K, 64, 27648, 5120) == KernelFamily::kTiledMfma);
  EXPECT(FusedQuantGemm::SelectKernel(Q4_K, 96, 27648, 5120) == KernelFamily::kF16DequantMfma);
  EXPECT(FusedQuantGemm::SelectKernel(Q6_K, 48, 5120, 27648) == KernelFamily::kF16DequantMfma);
  EXPECT(FusedQuantGemm::SelectKernel(Q8_0, 512, 64, 2080) == KernelFamily::kGemv);  // K % 64 != 0
  EXPECT(FusedQuantGemm::SelectKernel(Q8_0, 8, 64, 2080) == KernelFamily::kSkinnyMfma);
  EXPECT(FusedQuantGemm::SelectKernel(Q8_0, 40, 64, 2080) == KernelFamily::kGemv);
  EXPECT(FusedQuantGemm::SelectKernel(Q4_K, 1, 64, 100) == KernelFamily::kNone);
  EXPECT(std::string(FusedQuantGemm::KernelFamilyName(KernelFamily::kTiledMfma)) ==
         "tiled int8 MFMA");

  // rejected calls return false before any launch (no GPU needed)
  uint16_t dummy_out[4];
  const uint8_t dummy[64] = {};
  QuantizedWeightInfo w{dummy, Q4_K, 256};
  EXPECT(!FusedQuantGemm::GemvQ8_1(QuantizedWeightInfo{}, dummy, dummy_out, 1, 1, 256, nullptr));
  EXPECT(!FusedQuantGemm::GemvQ8_1(w, nullptr, dummy_out, 1, 1, 256, nullptr));
  EXPECT(!FusedQuantGemm::GemvQ8_1(w, dummy, nullptr, 1, 1, 256, nullptr));
  QuantizedWeightInfo bad_type{dummy, Q8_1, 256};
  EXPECT(!FusedQuantGemm::GemvQ8_1(bad_type, dummy, dummy_out, 1, 1, 256, nullptr));
  EXPECT(!FusedQuantGemm::GemvQ8_1(w, dummy, dummy_out, 0, 1, 256, nullptr));
  EXPECT(!FusedQuantGemm::GemvQ8_1(w, dummy, dummy_out, 1, 1, 100, nullptr));
  QuantizedWeightInfo small{dummy, Q4_K, 255};  // view smaller than N x K
  EXPECT(!FusedQuantGemm::GemvQ8_1(small, dummy, dummy_out, 1, 1, 256, nullptr));
  NativeExecutionPolicy off;
  off.disable_fused_gemv = true;
  EXPECT(!FusedQuantGemm::GemvQ8_1(w, dummy, dummy_out, 1, 1, 256, nullptr, &off));
  EXPECT(!FusedQuantGemm::GemvQ8_1AccumF32(w, dummy, reinterpret_cast<float *>(dummy_out), 1, 1,
                                           256, nullptr, &off));
  setenv("INFERFLUX_DISABLE_FUSED_GEMV", "1", 1);
  EXPECT(NativeExecutionPolicy::FromEnv().disable_fused_gemv);
  EXPECT(!FusedQuantGemm::GemvQ8_1(w, dummy, dummy_out, 1, 1, 256, nullptr));
  setenv("INFERFLUX_DISABLE_FUSED_GEMV", "off", 1);
  EXPECT(!NativeExecutionPolicy::FromEnv().disable_fused_gemv);
  unsetenv("INFERFLUX_DISABLE_FUSED_GEMV");
  // grouped: mixed quant types or a null output are not handled
  std::array<PackedProjectionSpec, 2> mixed{
      PackedProjectionSpec{QuantizedWeightInfo{dummy, Q4_K, 256}, dummy_out, 1},
      PackedProjectionSpec{QuantizedWeightInfo{dummy, Q6_K, 256}, dummy_out, 1}};
  EXPECT(!FusedQuantGemm::GemvQ8_1Pair(mixed, dummy, 1, 256, nullptr));
  mixed[1].weight.quant_type = Q4_K;
  mixed[1].output = nullptr;
  EXPECT(!FusedQuantGemm::GemvQ8_1Pair(mixed, dummy, 1, 256, nullptr));
  // packed activations: the reference's types only; a missing scale
  // vector, a disabled policy or mixed types are not handled
  EXPECT(FusedQuantGemm::SupportsPackedActivations(Q4_K));
  EXPECT(FusedQuantGemm::SupportsPackedActivations(Q8_0));
  EXPECT(!FusedQuantGemm::SupportsPackedActivations(13));
  const auto *codes = reinterpret_cast<const int8_t *>(dummy);
  const auto *scales = reinterpret_cast<const float *>(dummy);
  const PackedActivationInfo pa{codes, scales};
  EXPECT(!FusedQuantGemm::GemvPacked(QuantizedWeightInfo{dummy, 13, 256}, pa, dummy_out, 1, 1,
                                     256, nullptr));
  EXPECT(!FusedQuantGemm::GemvPacked(w, PackedActivationInfo{codes, nullptr}, dummy_out, 1, 1,
                                     256, nullptr));
  EXPECT(!FusedQuantGemm::GemvPacked(w, pa, dummy_out, 1, 1, 100, nullptr));
  EXPECT(!FusedQuantGemm::GemvPacked(w, pa, dummy_out, 1, 1, 256, nullptr, &off));
  mixed[1].output = dummy_out;
  mixed[1].weight.quant_type = Q6_K;
  EXPECT(!FusedQuantGemm::GemvPackedPair(mixed, pa, 1, 256, nullptr));
}

// ------------------------------------------------------------------- gpu
void TestGpuCase(int qtype, int M, int N, int K) {
  std::printf("[gpu] qtype=%d M=%d N=%d K=%d\n", qtype, M, N, K);
  std::fflush(stdout);
  Problem p = MakeProblem(qtype, M, N, K, 7 * qtype + M);
  hipStream_t s;
  HIP_OK(hipStreamCreate(&s));
  Dev dw(p.w.size()), dx(p.x.size() * 4), da(p.a.size()), dy(static_cast<size_t>(M) * N * 4),
      dh(static_cast<size_t>(M) * N * 2), db(static_cast<size_t>(N) * 2);
  HIP_OK(hipMemcpy(dw.p, p.w.data(), p.w.size(), hipMemcpyHostToDevice));
  HIP_OK(hipMemcpy(dx.p, p.x.data(), p.x.size() * 4, hipMemcpyHostToDevice));
  FusedQuantGemm::QuantizeRowQ8_1(dx.as<float>(), da.p, M, K, s);
  HIP_OK(hipStreamSynchronize(s));
  std::vector<uint8_t> a(p.a.size());
  HIP_OK(hipMemcpy(a.data(), da.p, a.size(), hipMemcpyDeviceToHost));
  EXPECT(a == p.a);  // Q8_1 codes and scales bit-exact

  const QuantizedWeightInfo w{dw.p, qtype, static_cast<int64_t>(N) * K};
  std::vector<float> y(static_cast<size_t>(M) * N);
  // fp32 store
  EXPECT(FusedQuantGemm::GemvQ8_1F32(w, da.p, dy.as<float>(), M, N, K, s));
  HIP_OK(hipStreamSynchronize(s));
  HIP_OK(hipMemcpy(y.data(), dy.p, y.size() * 4, hipMemcpyDeviceToHost));
  EXPECT(RowsClose(y, p.ye, M, N, 1e-3, false));
  // fp32 accumulate onto 0.5
  std::vector<float> base(y.size(), 0.5f);
  HIP_OK(hipMemcpy(dy.p, base.data(), base.size() * 4, hipMemcpyHostToDevice));
  EXPECT(FusedQuantGemm::GemvQ8_1AccumF32(w, da.p, dy.as<float>(), M, N, K, s));
  HIP_OK(hipStreamSynchronize(s));
  HIP_OK(hipMemcpy(y.data(), dy.p, y.size() * 4, hipMemcpyDeviceToHost));
  for (auto &v : y) v -= 0.5f;
  EXPECT(RowsClose(y, p.ye, M, N, 1e-3, false));
  // fp16 store
  std::vector<uint16_t> h(y.size());
  EXPECT(FusedQuantGemm::GemvQ8_1(w, da.p, dh.as<uint16_t>(), M, N, K, s));
  HIP_OK(hipStreamSynchronize(s));
  HIP_OK(hipMemcpy(h.data(), dh.p, h.size() * 2, hipMemcpyDeviceToHost));
  EXPECT(RowsClose(HalfToFloat(h), p.ye, M, N, 1e-3, true));
  // fp16 with bias, then fp16 accumulate of the same product
  std::vector<uint16_t> bias(N);
  std::vector<double> ye_b(p.ye);
  for (int n = 0; n < N; ++n) {
    bias[n] = orc_f32_to_f16(0.25f * static_cast<float>(n % 7) - 0.5f);
    for (int m = 0; m < M; ++m) ye_b[static_cast<size_t>(m) * N + n] += orc_f16_to_f32(bias[n]);
  }
  HIP_OK(hipMemcpy(db.p, bias.data(), bias.size() * 2, hipMemcpyHostToDevice));
  EXPECT(FusedQuantGemm::GemvQ8_1WithBias(w, da.p, dh.as<uint16_t>(), db.as<uint16_t>(), M, N, K,
                                          s));
  HIP_OK(hipStreamSynchronize(s));
  HIP_OK(hipMemcpy(h.data(), dh.p, h.size() * 2, hipMemcpyDeviceToHost));
  EXPECT(RowsClose(HalfToFloat(h), ye_b, M, N, 1e-3, true));
  EXPECT(FusedQuantGemm::GemvQ8_1Accum(w, da.p, dh.as<uint16_t>(), M, N, K, s));
  HIP_OK(hipStreamSynchronize(s));
  HIP_OK(hipMemcpy(h.data(), dh.p, h.size() * 2, hipMemcpyDeviceToHost));
  std::vector<double> ye_2(ye_b);
  for (size_t i = 0; i < ye_2.size(); ++i) ye_2[i] += p.ye[i];
  EXPECT(RowsClose(HalfToFloat(h), ye_2, M, N, 2e-3, true));
  HIP_OK(hipStreamDestroy(s));
}

// Exact-arithmetic cases of the fused producers (the randomized ones run
// from Python): x = +-1 with eps = 0 gives rms = 1; gate >= 20 gives
// silu(gate) = gate in fp32.
void TestProducers() {
  std::printf("[gpu producers]\n");
  std::fflush(stdout);
  const int M = 2, K = 1024;
  Rng r(77);
  std::vector<float> x(M * K), g(M * K), u(M * K);
  std::vector<uint16_t> w(K);
  for (auto &v : x) v = (r.next() & 1) ? 1.0f : -1.0f;
  for (auto &v : w) v = orc_f32_to_f16(r.normal());
  for (auto &v : g) v = 20.0f + static_cast<float>(r.next() % 20);
  for (auto &v : u) v = static_cast<float>(static_cast<int>(r.next() % 7) - 3);
  Dev dx(x.size() * 4), dw(w.size() * 2), dg(g.size() * 4), du(u.size() * 4),
      da(static_cast<size_t>(M) * (K / 32) * 36);
  HIP_OK(hipMemcpy(dx.p, x.data(), x.size() * 4, hipMemcpyHostToDevice));
  HIP_OK(hipMemcpy(dw.p, w.data(), w.size() * 2, hipMemcpyHostToDevice));
  HIP_OK(hipMemcpy(dg.p, g.data(), g.size() * 4, hipMemcpyHostToDevice));
  HIP_OK(hipMemcpy(du.p, u.data(), u.size() * 4, hipMemcpyHostToDevice));
  std::vector<uint8_t> a(static_cast<size_t>(M) * (K / 32) * 36), e(a.size());
  FusedQuantGemm::FusedRmsNormQuantizeQ8_1(dx.as<float>(), dw.as<uint16_t>(), da.p, M, K, 0.0f,
                                           nullptr);
  HIP_OK(hipDeviceSynchronize());
  HIP_OK(hipMemcpy(a.data(), da.p, a.size(), hipMemcpyDeviceToHost));
  orc_rmsnorm_quantize_q8_1(x.data(), w.data(), e.data(), M, K, 0.0f);
  EXPECT(a == e);
  FusedQuantGemm::SiluMulQuantizeQ8_1(dg.as<float>(), du.as<float>(), da.p, M, K, nullptr);
  HIP_OK(hipDeviceSynchronize());
  HIP_OK(hipMemcpy(a.data(), da.p, a.size(), hipMemcpyDeviceToHost));
  orc_silu_mul_quantize_q8_1(g.data(), u.data(), e.data(), M, K);
  EXPECT(a == e);
}

template <size_t C>
void TestGrouped(int qtype, int M, int K, const std::array<int, C> &Ns) {
  std::printf("[gpu grouped x%zu] qtype=%d M=%d K=%d\n", C, qtype, M, K);
  std::fflush(stdout);
  std::vector<Problem> ps;
  for (size_t i = 0; i < C; ++i) ps.push_back(MakeProblem(qtype, M, Ns[i], K, 100 + i));
  // all projections read projection 0's activations
  std::vector<std::unique_ptr<Dev>> dws, dys;
  Dev da(ps[0].a.size());
  HIP_OK(hipMemcpy(da.p, ps[0].a.data(), ps[0].a.size(), hipMemcpyHostToDevice));
  std::array<PackedProjectionSpec, C> spec{};
  for (size_t i = 0; i < C; ++i) {
    dws.emplace_back(new Dev(ps[i].w.size()));
    dys.emplace_back(new Dev(static_cast<size_t>(M) * Ns[i] * 2));
    HIP_OK(hipMemcpy(dws[i]->p, ps[i].w.data(), ps[i].w.size(), hipMemcpyHostToDevice));
    spec[i] = PackedProjectionSpec{QuantizedWeightInfo{dws[i]->p, qtype, int64_t{Ns[i]} * K},
                                   dys[i]->template as<uint16_t>(), Ns[i]};
  }
  bool ok;
  if constexpr (C == 2) ok = FusedQuantGemm::GemvQ8_1Pair(spec, da.p, M, K, nullptr);
  else ok = FusedQuantGemm::GemvQ8_1Triple(spec, da.p, M, K, nullptr);
  EXPECT(ok);
  HIP_OK(hipDeviceSynchronize());
  for (size_t i = 0; i < C; ++i) {
    std::vector<double> ye(static_cast<size_t>(M) * Ns[i]);
    orc_gemv_exact(qtype, ps[i].w.data(), ps[0].a.data(), ye.data(), M, Ns[i], K, 8);
    std::vector<uint16_t> h(ye.size());
    HIP_OK(hipMemcpy(h.data(), dys[i]->p, h.size() * 2, hipMemcpyDeviceToHost));
    EXPECT(RowsClose(HalfToFloat(h), ye, M, Ns[i], 1e-3, true));
  }
}

// Packed activations: QuantizeRowsSymmetric on fp16 rows (bit-exact with
// the oracle) feeding GemvPacked / Pair / Triple (fp16 out, oracle fp64).
template <size_t C>
void TestPacked(int qtype, int M, int K, const std::array<int, C> &Ns) {
  std::printf("[gpu packed x%zu] qtype=%d M=%d K=%d\n", C, qtype, M, K);
  std::fflush(stdout);
  Rng r(7 + M + K);
  std::vector<uint16_t> xh(static_cast<size_t>(M) * K);
  std::vector<float> xf(xh.size());
  for (size_t i = 0; i < xh.size(); ++i) {
    xh[i] = orc_f32_to_f16(r.normal());
    xf[i] = orc_f16_to_f32(xh[i]);
  }
  Dev dx(xh.size() * 2), dc(xh.size()), ds(static_cast<size_t>(M) * 4);
  HIP_OK(hipMemcpy(dx.p, xh.data(), xh.size() * 2, hipMemcpyHostToDevice));
  EXPECT(FusedQuantGemm::QuantizeRowsSymmetric(dx.as<uint16_t>(), dc.as<int8_t>(), ds.as<float>(),
                                               M, K, nullptr));
  HIP_OK(hipDeviceSynchronize());
  std::vector<int8_t> c(xh.size()), ce(xh.size());
  std::vector<float> sc(M), se(M);
  HIP_OK(hipMemcpy(c.data(), dc.p, c.size(), hipMemcpyDeviceToHost));
  HIP_OK(hipMemcpy(sc.data(), ds.p, sc.size() * 4, hipMemcpyDeviceToHost));
  orc_quantize_rows_symmetric(xf.data(), ce.data(), se.data(), M, K);
  EXPECT(c == ce);
  EXPECT(std::memcmp(sc.data(), se.data(), sc.size() * 4) == 0);
  std::vector<std::vector<uint8_t>> ws;
  std::vector<std::unique_ptr<Dev>> dws, dys;
  std::array<PackedProjectionSpec, C> spec{};
  for (size_t i = 0; i < C; ++i) {
    ws.push_back(MakeBlocks(qtype, Ns[i], K, 300 + i));
    dws.emplace_back(new Dev(ws[i].size()));
    dys.emplace_back(new Dev(static_cast<size_t>(M) * Ns[i] * 2));
    HIP_OK(hipMemcpy(dws[i]->p, ws[i].data(), ws[i].size(), hipMemcpyHostToDevice));
    spec[i] = PackedProjectionSpec{QuantizedWeightInfo{dws[i]->p, qtype, int64_t{Ns[i]} * K},
                                   dys[i]->template as<uint16_t>(), Ns[i]};
  }
  const PackedActivationInfo act{dc.as<int8_t>(), ds.as<float>()};
  bool ok;
  if constexpr (C == 1)
    ok = FusedQuantGemm::GemvPacked(spec[0].weight, act, spec[0].output, M, Ns[0], K, nullptr);
  else if constexpr (C == 2) ok = FusedQuantGemm::GemvPackedPair(spec, act, M, K, nullptr);
  else ok = FusedQuantGemm::GemvPackedTriple(spec, act, M, K, nullptr);
  EXPECT(ok);
  HIP_OK(hipDeviceSynchronize());
  for (size_t i = 0; i < C; ++i) {
    std::vector<double> ye(static_cast<size_t>(M) * Ns[i]);
    orc_gemv_packed_exact(qtype, ws[i].data(), c.data(), sc.data(), ye.data(), M, Ns[i], K, 8);
    std::vector<uint16_t> h(ye.size());
    HIP_OK(hipMemcpy(h.data(), dys[i]->p, h.size() * 2, hipMemcpyDeviceToHost));
    EXPECT(RowsClose(HalfToFloat(h), ye, M, Ns[i], 1e-3, true));
  }
}

}  // namespace

int main(int argc, char **argv) {
  const std::string mode = argc > 1 ? argv[1] : "policy";
  if (mode == "policy") {
    TestPolicy();
  } else if (mode == "gpu") {
    TestGpuCase(Q4_K, 1, 300, 2048);
    TestGpuCase(Q6_K, 2, 129, 1024);
    TestGpuCase(Q8_0, 1, 77, 2080);
    TestGpuCase(Q4_K, 5, 200, 1024);
    TestGpuCase(Q6_K, 24, 96, 2048);
    TestGpuCase(Q8_0, 40, 160, 512);
    TestGpuCase(13, 1, 300, 2048);  // Q5_K
    TestGpuCase(13, 7, 130, 1024);
    TestGpuCase(15, 2, 200, 1024);  // Q8_K
    TestGpuCase(15, 64, 70, 512);
    TestProducers();
    TestGrouped<2>(Q4_K, 1, 2048, {300, 173});
    TestGrouped<3>(Q4_K, 2, 1024, {128, 64, 65});
    TestGrouped<3>(Q6_K, 1, 512, {33, 1, 250});
    TestGrouped<2>(Q8_0, 4, 256, {70, 90});
    TestPacked<1>(Q4_K, 1, 2048, {300});
    TestPacked<2>(Q6_K, 2, 256, {8, 6});
    TestPacked<3>(Q4_K, 2, 256, {8, 6, 4});
    TestPacked<2>(Q8_0, 3, 1056, {70, 33});
    TestPacked<1>(15, 2, 1024, {100});  // Q8_K
  } else {
    std::printf("usage: %s policy|gpu\n", argv[0]);
    return 2;
  }
  std::printf("%s: %d failure(s)\n", mode.c_str(), g_failures);
  return g_failures ? 1 : 0;
}
