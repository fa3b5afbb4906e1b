// ifx_gguf_model.h -- C++ host mirror of the reference's GGUF model loader
// and raw quantized-weight map, over the C ABI of ifx_gguf.h.
//
//  GgufModelLoader  ~ GGUFModelLoader (runtime/backends/cuda/native/
//                     gguf_model_loader.h; Load :284-349, model info
//                     :529-604 and :903-985, UploadToGPU :1005-1047,
//                     FreeGPUMemory :1056-1072, GetGPUBuffer/GetGPUSize
//                     :1074-1076)
//  QuantizedWeightMap ~ the raw accessors of QuantizedWeightMap
//                     (quantized_weight_map.cpp:379-434 and :482, tied LM
//                     head :81-86): per-layer QuantizedWeightInfo views of
//                     the uploaded blocks, the W argument of FusedQuantGemm.
//
// Same names and bool convention as the reference (false = failed, the
// reason in last_status()).  The upload allocates one device buffer for
// every tensor (256-byte aligned tensors), as UploadToGPU's single
// cudaMalloc does; nothing else allocates device memory.
#ifndef IFX_GGUF_MODEL_H
#define IFX_GGUF_MODEL_H

#include <hip/hip_runtime_api.h>

#include <cstdint>
#include <string>
#include <unordered_map>
#include <vector>

#include "ifx_fused_quant_gemm.h"
#include "ifx_gguf.h"

namespace inferflux {
namespace rocm {

// The hyperparameters the reference extracts (model_loader.h ModelInfo subset).
struct GgufModelInfo {
  std::string model_type;
  int num_hidden_layers{0};
  int hidden_size{0};
  int intermediate_size{0};
  int num_attention_heads{0};
  int num_key_value_heads{0};
  int max_position_embeddings{0};
  int vocab_size{0};
  float rope_freq_base{0.0f};
  float rms_norm_eps{0.0f};
};

struct GgufTensorView {
  std::string name;
  int type{-1};
  std::vector<int64_t> shape;  // ne[0] first
  uint64_t byte_size{0};
  const void *host_data{nullptr};  // into the file mapping
  const void *gpu_data{nullptr};   // after UploadToGPU
  int64_t num_elements() const;
};

class GgufModelLoader {
 public:
  GgufModelLoader() = default;
  ~GgufModelLoader();
  GgufModelLoader(const GgufModelLoader &) = delete;
  GgufModelLoader &operator=(const GgufModelLoader &) = delete;

  bool Load(const std::string &path);
  bool UploadToGPU(hipStream_t stream);
  void FreeGPUMemory();

  const GgufModelInfo &GetModelInfo() const { return info_; }
  std::vector<std::string> GetTensorNames() const;
  const GgufTensorView *GetTensorByGGUFName(const std::string &name) const;
  void *GetGPUBuffer() const { return d_buffer_; }
  size_t GetGPUSize() const { return d_bytes_; }
  const ifx_gguf *handle() const { return g_; }
  int last_status() const { return status_; }

 private:
  void Reset();
  ifx_gguf *g_{nullptr};
  GgufModelInfo info_;
  std::vector<GgufTensorView> tensors_;
  std::unordered_map<std::string, size_t> by_name_;
  void *d_buffer_{nullptr};
  size_t d_bytes_{0};
  int status_{0};
};

class QuantizedWeightMap {
 public:
  explicit QuantizedWeightMap(const GgufModelLoader &loader) : loader_(loader) {}
  int NumLayers() const { return loader_.GetModelInfo().num_hidden_layers; }
  QuantizedWeightInfo LayerQProjRaw(int layer) const { return Raw(layer, "attn_q"); }
  QuantizedWeightInfo LayerKProjRaw(int layer) const { return Raw(layer, "attn_k"); }
  QuantizedWeightInfo LayerVProjRaw(int layer) const { return Raw(layer, "attn_v"); }
  QuantizedWeightInfo LayerOProjRaw(int layer) const { return Raw(layer, "attn_output"); }
  QuantizedWeightInfo LayerGateProjRaw(int layer) const { return Raw(layer, "ffn_gate"); }
  QuantizedWeightInfo LayerUpProjRaw(int layer) const { return Raw(layer, "ffn_up"); }
  QuantizedWeightInfo LayerDownProjRaw(int layer) const { return Raw(layer, "ffn_down"); }
  QuantizedWeightInfo LmHeadRaw() const;
  bool HasQuantizedWeights() const;

 private:
  QuantizedWeightInfo Raw(int layer, const char *component) const;
  static QuantizedWeightInfo Info(const GgufTensorView *t);
  const GgufModelLoader &loader_;
};

}  // namespace rocm
}  // namespace inferflux

#endif  // IFX_GGUF_MODEL_H
