// gguf_model.cpp -- GgufModelLoader / QuantizedWeightMap (ifx_gguf_model.h).
#include "ifx_gguf_model.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstring>
#include <limits>

namespace inferflux {
namespace rocm {

namespace {

constexpr uint64_t kDeviceAlign = 256;

int Saturate(int64_t v) {
  return static_cast<int>(std::min<int64_t>(std::max<int64_t>(v, 0),
                                            std::numeric_limits<int>::max()));
}

int64_t GetInt(const ifx_gguf *g, const std::string &key, int64_t dflt) {
  int64_t v = 0;
  return ifx_gguf_get_int(g, key.c_str(), &v) == IFX_GGUF_OK ? v : dflt;
}

double GetFloat(const ifx_gguf *g, const std::string &key, double dflt) {
  double v = 0;
  return ifx_gguf_get_float(g, key.c_str(), &v) == IFX_GGUF_OK ? v : dflt;
}

}  // namespace

int64_t GgufTensorView::num_elements() const {
  int64_t n = 1;
  for (int64_t d : shape) n *= d;
  return n;
}

GgufModelLoader::~GgufModelLoader() { Reset(); }

void GgufModelLoader::Reset() {
  FreeGPUMemory();
  if (g_) ifx_gguf_close(g_);
  g_ = nullptr;
  info_ = GgufModelInfo{};
  tensors_.clear();
  by_name_.clear();
}

// gguf_model_loader.cpp:284-349 (+ the model info of :529-604, :903-985).
bool GgufModelLoader::Load(const std::string &path) {
  Reset();
  status_ = ifx_gguf_open(path.c_str(), &g_);
  if (status_ != IFX_GGUF_OK) {
    g_ = nullptr;
    return false;
  }
  const int64_t n = ifx_gguf_n_tensors(g_);
  tensors_.reserve(static_cast<size_t>(n));
  for (int64_t i = 0; i < n; ++i) {
    ifx_gguf_tensor t{};
    ifx_gguf_tensor_info(g_, i, &t);
    GgufTensorView v;
    v.name = t.name;
    v.type = t.type;
    v.shape.assign(t.shape, t.shape + t.n_dims);
    v.byte_size = t.byte_size;
    v.host_data = t.host_data;
    by_name_[v.name] = tensors_.size();
    tensors_.push_back(std::move(v));
  }

  const char *arch = nullptr;
  uint64_t arch_len = 0;
  if (ifx_gguf_get_string(g_, "general.architecture", &arch, &arch_len) == IFX_GGUF_OK)
    info_.model_type.assign(arch, arch_len);
  const std::string p = info_.model_type + ".";
  info_.num_hidden_layers = Saturate(GetInt(g_, p + "block_count", 0));
  info_.hidden_size = Saturate(GetInt(g_, p + "embedding_length", 0));
  info_.intermediate_size = Saturate(GetInt(g_, p + "feed_forward_length", 0));
  info_.num_attention_heads = Saturate(GetInt(g_, p + "attention.head_count", 0));
  info_.num_key_value_heads = Saturate(GetInt(g_, p + "attention.head_count_kv", 0));
  info_.max_position_embeddings = Saturate(GetInt(g_, p + "context_length", 0));
  info_.rope_freq_base = static_cast<float>(GetFloat(g_, p + "rope.freq_base", 0.0));
  info_.rms_norm_eps = static_cast<float>(GetFloat(g_, p + "attention.layer_norm_rms_epsilon", 0.0));
  if (info_.num_key_value_heads <= 0) info_.num_key_value_heads = info_.num_attention_heads;
  if (info_.rms_norm_eps <= 0.0f) info_.rms_norm_eps = 1e-6f;
  const GgufTensorView *emb = GetTensorByGGUFName("tok_emb.weight");
  if (!emb) emb = GetTensorByGGUFName("token_embd.weight");
  if (emb && emb->shape.size() >= 2) {
    info_.vocab_size = Saturate(std::max(emb->shape[0], emb->shape[1]));
    if (info_.hidden_size <= 0) info_.hidden_size = Saturate(std::min(emb->shape[0], emb->shape[1]));
  } else if (emb) {
    info_.vocab_size = Saturate(emb->shape[0]);
  }
  return true;
}

// gguf_model_loader.cpp:1005-1047: one buffer, every tensor copied in.
bool GgufModelLoader::UploadToGPU(hipStream_t stream) {
  if (!g_) {
    status_ = IFX_GGUF_ARGUMENT;
    return false;
  }
  FreeGPUMemory();
  const uint64_t bytes = ifx_gguf_device_bytes(g_, kDeviceAlign);
  if (bytes == 0) return true;  // no tensors
  hipError_t e = hipMalloc(&d_buffer_, bytes);
  if (e != hipSuccess) {
    d_buffer_ = nullptr;
    status_ = -static_cast<int>(e);
    return false;
  }
  d_bytes_ = bytes;
  std::vector<uint64_t> offs(tensors_.size());
  status_ = ifx_gguf_upload(g_, d_buffer_, bytes, kDeviceAlign, offs.data(), stream);
  if (status_ != IFX_GGUF_OK) {
    FreeGPUMemory();
    return false;
  }
  for (size_t i = 0; i < tensors_.size(); ++i)
    tensors_[i].gpu_data = static_cast<const uint8_t *>(d_buffer_) + offs[i];
  return true;
}

void GgufModelLoader::FreeGPUMemory() {
  if (d_buffer_) (void)hipFree(d_buffer_);
  d_buffer_ = nullptr;
  d_bytes_ = 0;
  for (auto &t : tensors_) t.gpu_data = nullptr;
}

std::vector<std::string> GgufModelLoader::GetTensorNames() const {
  std::vector<std::string> out;
  out.reserve(tensors_.size());
  for (const auto &t : tensors_) out.push_back(t.name);
  return out;
}

const GgufTensorView *GgufModelLoader::GetTensorByGGUFName(const std::string &name) const {
  auto it = by_name_.find(name);
  return it == by_name_.end() ? nullptr : &tensors_[it->second];
}

// quantized_weight_map.cpp:378-392 MakeRawInfo: quantized tensors only.
QuantizedWeightInfo QuantizedWeightMap::Info(const GgufTensorView *t) {
  QuantizedWeightInfo info;
  if (!t || t->type == 0 || t->type == 1 || !t->gpu_data) return info;
  info.data = t->gpu_data;
  info.quant_type = t->type;
  info.num_elements = t->num_elements();
  return info;
}

QuantizedWeightInfo QuantizedWeightMap::Raw(int layer, const char *component) const {
  if (layer < 0 || layer >= NumLayers()) return {};
  const std::string base = "blk." + std::to_string(layer) + ".";
  const GgufTensorView *t = loader_.GetTensorByGGUFName(base + component + ".weight");
  if (!t && std::strcmp(component, "attn_output") == 0)  // gguf_util.cpp:294
    t = loader_.GetTensorByGGUFName(base + "attn_o.weight");
  return Info(t);
}

// quantized_weight_map.cpp:81-86, 482: output.weight, else tied embeddings.
QuantizedWeightInfo QuantizedWeightMap::LmHeadRaw() const {
  for (const char *name : {"output.weight", "lm_head.weight", "token_embd.weight", "tok_emb.weight"}) {
    const GgufTensorView *t = loader_.GetTensorByGGUFName(name);
    if (t) return Info(t);
  }
  return {};
}

bool QuantizedWeightMap::HasQuantizedWeights() const {
  for (const auto &name : loader_.GetTensorNames()) {
    const GgufTensorView *t = loader_.GetTensorByGGUFName(name);
    if (t && t->type != 0 && t->type != 1) return true;
  }
  return false;
}

}  // namespace rocm
}  // namespace inferflux
