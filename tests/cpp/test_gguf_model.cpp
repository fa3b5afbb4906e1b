// test_gguf_model.cpp -- tests of the C++ GGUF loader mirror
// (include/ifx_gguf_model.h) on a file written by tests/gguf_writer.py.
//
//   test_gguf_model cpu <file>   parse, model info, names, tied LM head
//   test_gguf_model gpu <file>   upload, weight views, one FusedQuantGemm
//                                GEMV on a loaded projection vs the oracle
// The file is the 2-layer model of tests/test_gguf.py::model_tensors.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdio>
#include <cstring>
#include <random>
#include <string>
#include <vector>

#include "../../include/ifx_fused_quant_gemm.h"
#include "../../include/ifx_gguf_model.h"

extern "C" {
int orc_quantize_q8_1_f32(const float *x, void *out, int64_t M, int64_t K);
int orc_gemv_exact(int qtype, const void *W, const void *A, double *y, int M, int N, int K,
                   int threads);
}

using inferflux::rocm::FusedQuantGemm;
using inferflux::rocm::GgufModelLoader;
using inferflux::rocm::QuantizedWeightInfo;
using inferflux::rocm::QuantizedWeightMap;

namespace {

int g_failures = 0;

#define EXPECT(cond)                                                  \
  do {                                                                \
    if (!(cond)) {                                                    \
      std::printf("  FAILED %s:%d: %s\n", __FILE__, __LINE__, #cond); \
      ++g_failures;                                                   \
    }                                                                 \
  } while (0)

void TestCpu(const std::string &path) {
  GgufModelLoader loader;
  EXPECT(!loader.Load(path + ".missing"));
  EXPECT(loader.last_status() == IFX_GGUF_IO);
  EXPECT(loader.GetTensorNames().empty());
  EXPECT(!loader.UploadToGPU(nullptr));  // nothing loaded
  EXPECT(loader.Load(path));
  const auto &info = loader.GetModelInfo();
  EXPECT(info.model_type == "qwen2");
  EXPECT(info.num_hidden_layers == 2 && info.hidden_size == 512 && info.intermediate_size == 1024);
  EXPECT(info.num_attention_heads == 8 && info.num_key_value_heads == 2);
  EXPECT(info.vocab_size == 1000 && info.max_position_embeddings == 32768);
  EXPECT(std::fabs(info.rms_norm_eps - 1e-5f) < 1e-9f && info.rope_freq_base == 1e6f);
  EXPECT(loader.GetTensorNames().size() == 18);
  const auto *down = loader.GetTensorByGGUFName("blk.1.ffn_down.weight");
  EXPECT(down && down->type == 14 && down->shape.size() == 2 && down->shape[0] == 1024 &&
         down->shape[1] == 512 && down->byte_size == 512u * 4 * 210 && down->host_data);
  EXPECT(down && down->num_elements() == 1024 * 512);
  EXPECT(loader.GetTensorByGGUFName("blk.9.ffn_down.weight") == nullptr);
  EXPECT(loader.GetGPUBuffer() == nullptr && loader.GetGPUSize() == 0);
  QuantizedWeightMap map(loader);
  EXPECT(map.NumLayers() == 2 && map.HasQuantizedWeights());
  // views exist only after the upload
  EXPECT(map.LayerQProjRaw(0).data == nullptr);
  EXPECT(map.LayerQProjRaw(-1).quant_type == -1 && map.LayerQProjRaw(2).quant_type == -1);
  std::printf("cpu: %d failure(s)\n", g_failures);
}

void TestGpu(const std::string &path) {
  GgufModelLoader loader;
  EXPECT(loader.Load(path));
  hipStream_t s;
  (void)hipStreamCreate(&s);
  EXPECT(loader.UploadToGPU(s));
  EXPECT(loader.GetGPUBuffer() != nullptr && loader.GetGPUSize() % 256 == 0);
  QuantizedWeightMap map(loader);
  // every view holds the file's bytes, 256-byte aligned
  for (const auto &name : loader.GetTensorNames()) {
    const auto *t = loader.GetTensorByGGUFName(name);
    std::vector<uint8_t> back(t->byte_size);
    (void)hipMemcpy(back.data(), t->gpu_data, t->byte_size, hipMemcpyDeviceToHost);
    EXPECT(reinterpret_cast<uintptr_t>(t->gpu_data) % 256 == 0);
    EXPECT(std::memcmp(back.data(), t->host_data, t->byte_size) == 0);
  }
  const QuantizedWeightInfo gate = map.LayerGateProjRaw(1), o = map.LayerOProjRaw(0);
  EXPECT(gate.data && gate.quant_type == 12 && gate.num_elements == 1024 * 512);
  EXPECT(o.data && o.quant_type == 12);
  const QuantizedWeightInfo head = map.LmHeadRaw();  // tied: token_embd (Q8_0)
  EXPECT(head.data && head.quant_type == 8 && head.num_elements == 512 * 1000);
  // GEMV on the loaded gate projection, M = 2
  const int M = 2, N = 1024, K = 512;
  std::mt19937 rng(7);
  std::normal_distribution<float> nd;
  std::vector<float> x(M * K);
  for (float &v : x) v = nd(rng);
  std::vector<uint8_t> a(M * (K / 32) * 36);
  orc_quantize_q8_1_f32(x.data(), a.data(), M, K);
  void *da = nullptr;
  float *dy = nullptr;
  (void)hipMalloc(&da, a.size());
  (void)hipMalloc(&dy, M * N * sizeof(float));
  (void)hipMemcpy(da, a.data(), a.size(), hipMemcpyHostToDevice);
  EXPECT(FusedQuantGemm::GemvQ8_1F32(gate, da, dy, M, N, K, s));
  (void)hipStreamSynchronize(s);
  std::vector<float> y(M * N);
  (void)hipMemcpy(y.data(), dy, y.size() * sizeof(float), hipMemcpyDeviceToHost);
  std::vector<double> ye(M * N);
  orc_gemv_exact(12, loader.GetTensorByGGUFName("blk.1.ffn_gate.weight")->host_data, a.data(),
                 ye.data(), M, N, K, 4);
  for (int m = 0; m < M; ++m) {
    double err = 0, nrm = 0;
    for (int n = 0; n < N; ++n) {
      err = std::fmax(err, std::fabs(y[m * N + n] - ye[m * N + n]));
      nrm += ye[m * N + n] * ye[m * N + n];
    }
    EXPECT(err <= 1e-3 * std::sqrt(nrm));
  }
  loader.FreeGPUMemory();
  EXPECT(loader.GetGPUBuffer() == nullptr && map.LayerGateProjRaw(1).data == nullptr);
  (void)hipFree(da);
  (void)hipFree(dy);
  (void)hipStreamDestroy(s);
  std::printf("gpu: %d failure(s)\n", g_failures);
}

}  // namespace

int main(int argc, char **argv) {
  if (argc < 3) {
    std::printf("usage: %s cpu|gpu <file.gguf>\n", argv[0]);
    return 2;
  }
  const std::string mode = argv[1];
  if (mode == "cpu") TestCpu(argv[2]);
  else if (mode == "gpu") TestGpu(argv[2]);
  else return 2;
  return g_failures ? 1 : 0;
}
