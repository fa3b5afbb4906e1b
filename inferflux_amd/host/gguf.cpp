// gguf.cpp -- GGUF v2/v3 parser and device uploader (C ABI of ifx_gguf.h).
//
// Accept/reject rules follow the reference loader:
//  header  gguf_model_loader.cpp:351-374 + gguf_util.cpp:402-421 (magic,
//          version 0/1 legacy and > 3 rejected, negative counts rejected);
//  strings gguf_util.cpp:87-104 (u64 length, at most 1 GiB);
//  values  gguf_util.cpp:106-215 (unknown value types rejected);
//  alignment gguf_model_loader.cpp:418-448 (u32/u64 only, non-zero power of
//          two; default 32);
//  tensors gguf_model_loader.cpp:763-848 (1..8 dims, every dim > 0, type id
//          <= 15 and a known block size, u64 offset; a repeated name replaces
//          the earlier entry, as the reference's map assignment does);
//  data    gguf_model_loader.cpp:850-901 (data section at the aligned end of
//          the metadata; every tensor's bytes must be inside the file).
// The file is memory-mapped and parsed with a bounds-checked cursor.
#include "ifx_gguf.h"

#include <hip/hip_runtime.h>

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cstring>
#include <string>
#include <unordered_map>
#include <vector>

namespace {

constexpr uint32_t kMagic = 0x46554747;  // "GGUF" little-endian
constexpr uint32_t kMaxVersion = 3;
constexpr uint64_t kMaxString = 1ull << 30;
constexpr int kMaxDims = 8;
constexpr int kMaxArrayDepth = 4;

struct KV {
  std::string key;
  uint32_t type;
  uint64_t pos;        // first byte of the value in the mapping
  uint32_t elem_type;  // arrays
  uint64_t count;      // arrays
  uint64_t first_elem; // arrays: position of element 0
  std::vector<uint64_t> str_pos;  // string arrays: length-prefix position of each element
};

struct Tensor {
  std::string name;
  int type;
  int n_dims;
  int64_t shape[kMaxDims];
  uint64_t offset;
  uint64_t bytes;
};

// Block geometry of GGML tensor types (gguf_util.cpp:549-566).
bool type_block(int type, uint64_t *elems, uint64_t *bytes) {
  switch (type) {
  case 0: *elems = 1; *bytes = 4; return true;     // F32
  case 1: *elems = 1; *bytes = 2; return true;     // F16
  case 2: *elems = 32; *bytes = 18; return true;   // Q4_0
  case 3: *elems = 32; *bytes = 20; return true;   // Q4_1
  case 6: *elems = 32; *bytes = 22; return true;   // Q5_0
  case 7: *elems = 32; *bytes = 24; return true;   // Q5_1
  case 8: *elems = 32; *bytes = 34; return true;   // Q8_0
  case 9: *elems = 32; *bytes = 36; return true;   // Q8_1
  case 10: *elems = 256; *bytes = 96; return true; // Q2_K
  case 11: *elems = 256; *bytes = 110; return true; // Q3_K
  case 12: *elems = 256; *bytes = 144; return true; // Q4_K
  case 13: *elems = 256; *bytes = 176; return true; // Q5_K
  case 14: *elems = 256; *bytes = 210; return true; // Q6_K
  case 15: *elems = 256; *bytes = 292; return true; // Q8_K
  default: return false;
  }
}

uint64_t fixed_size(uint32_t vt) {
  switch (vt) {
  case IFX_GGUF_U8: case IFX_GGUF_I8: case IFX_GGUF_BOOL: return 1;
  case IFX_GGUF_U16: case IFX_GGUF_I16: return 2;
  case IFX_GGUF_U32: case IFX_GGUF_I32: case IFX_GGUF_F32: return 4;
  case IFX_GGUF_U64: case IFX_GGUF_I64: case IFX_GGUF_F64: return 8;
  default: return 0;
  }
}

class Cursor {
 public:
  Cursor(const uint8_t *p, uint64_t n) : p_(p), n_(n) {}
  uint64_t pos() const { return pos_; }
  bool skip(uint64_t k) {
    if (k > n_ - pos_) return false;
    pos_ += k;
    return true;
  }
  template <typename T>
  bool read(T *out) {
    if (sizeof(T) > n_ - pos_) return false;
    std::memcpy(out, p_ + pos_, sizeof(T));
    pos_ += sizeof(T);
    return true;
  }
  // u64 length + bytes; *at = position of the first byte
  bool string(uint64_t *at, uint64_t *len, int *err) {
    if (!read(len)) { *err = IFX_GGUF_TRUNCATED; return false; }
    if (*len > kMaxString) { *err = IFX_GGUF_BAD_KV; return false; }
    *at = pos_;
    if (!skip(*len)) { *err = IFX_GGUF_TRUNCATED; return false; }
    return true;
  }

 private:
  const uint8_t *p_;
  uint64_t n_;
  uint64_t pos_ = 0;
};

// Skips one value of type vt (gguf_util.cpp:173-215).
int skip_value(Cursor &c, uint32_t vt, int depth) {
  const uint64_t fs = fixed_size(vt);
  if (fs) return c.skip(fs) ? IFX_GGUF_OK : IFX_GGUF_TRUNCATED;
  if (vt == IFX_GGUF_STRING) {
    uint64_t at, len;
    int err = IFX_GGUF_OK;
    return c.string(&at, &len, &err) ? IFX_GGUF_OK : err;
  }
  if (vt == IFX_GGUF_ARRAY) {
    if (depth >= kMaxArrayDepth) return IFX_GGUF_BAD_KV;
    uint32_t et;
    uint64_t n;
    if (!c.read(&et) || !c.read(&n)) return IFX_GGUF_TRUNCATED;
    const uint64_t efs = fixed_size(et);
    if (efs) {
      if (n > UINT64_MAX / efs) return IFX_GGUF_BAD_KV;
      return c.skip(n * efs) ? IFX_GGUF_OK : IFX_GGUF_TRUNCATED;
    }
    if (et != IFX_GGUF_STRING && et != IFX_GGUF_ARRAY) return IFX_GGUF_BAD_KV;
    for (uint64_t i = 0; i < n; ++i) {
      const int r = skip_value(c, et, depth + 1);
      if (r) return r;
    }
    return IFX_GGUF_OK;
  }
  return IFX_GGUF_BAD_KV;  // unknown value type
}

bool is_pow2(uint64_t v) { return v && !(v & (v - 1)); }

uint64_t align_up(uint64_t v, uint64_t a) { return (v + a - 1) & ~(a - 1); }

}  // namespace

struct ifx_gguf {
  int fd = -1;
  const uint8_t *map = nullptr;
  uint64_t size = 0;
  uint32_t version = 0;
  uint64_t alignment = 32;
  uint64_t data_offset = 0;
  std::vector<KV> kvs;
  std::unordered_map<std::string, size_t> kv_index;
  std::vector<Tensor> tensors;
  std::unordered_map<std::string, int64_t> tensor_index;

  ~ifx_gguf() {
    if (map && size) munmap(const_cast<uint8_t *>(map), size);
    if (fd >= 0) close(fd);
  }
  const KV *kv(const char *key) const {
    if (!key) return nullptr;
    auto it = kv_index.find(key);
    return it == kv_index.end() ? nullptr : &kvs[it->second];
  }
};

namespace {

int parse(ifx_gguf *g) {
  Cursor c(g->map, g->size);
  uint32_t magic = 0;
  int64_t n_tensors = 0, n_kv = 0;
  if (!c.read(&magic)) return IFX_GGUF_TRUNCATED;
  if (magic != kMagic) return IFX_GGUF_BAD_MAGIC;
  if (!c.read(&g->version)) return IFX_GGUF_TRUNCATED;
  if (g->version <= 1 || g->version > kMaxVersion) return IFX_GGUF_BAD_VERSION;
  if (!c.read(&n_tensors) || !c.read(&n_kv)) return IFX_GGUF_TRUNCATED;
  if (n_tensors < 0 || n_kv < 0) return IFX_GGUF_BAD_KV;

  for (int64_t i = 0; i < n_kv; ++i) {
    KV kv{};
    uint64_t at, len;
    int err = IFX_GGUF_OK;
    if (!c.string(&at, &len, &err)) return err;
    kv.key.assign(reinterpret_cast<const char *>(g->map + at), len);
    if (!c.read(&kv.type)) return IFX_GGUF_TRUNCATED;
    kv.pos = c.pos();
    if (kv.type == IFX_GGUF_ARRAY) {
      Cursor peek = c;
      if (!peek.read(&kv.elem_type) || !peek.read(&kv.count)) return IFX_GGUF_TRUNCATED;
      kv.first_elem = peek.pos();
    }
    if (kv.key == "general.alignment") {
      uint64_t a = 0;
      if (kv.type == IFX_GGUF_U32) {
        uint32_t v;
        Cursor peek = c;
        if (!peek.read(&v)) return IFX_GGUF_TRUNCATED;
        a = v;
      } else if (kv.type == IFX_GGUF_U64) {
        Cursor peek = c;
        if (!peek.read(&a)) return IFX_GGUF_TRUNCATED;
      } else {
        return IFX_GGUF_BAD_KV;
      }
      if (!is_pow2(a)) return IFX_GGUF_BAD_KV;
      g->alignment = a;
    }
    if (kv.key == "general.architecture" && kv.type != IFX_GGUF_STRING) return IFX_GGUF_BAD_KV;
    if (kv.type == IFX_GGUF_ARRAY && kv.elem_type == IFX_GGUF_STRING) {
      // walk the elements here, keeping where each starts
      if (!c.skip(kv.first_elem - c.pos())) return IFX_GGUF_TRUNCATED;
      if (kv.count > (g->size - c.pos()) / 8) return IFX_GGUF_TRUNCATED;  // >= 8 bytes each
      kv.str_pos.reserve(kv.count);
      for (uint64_t e = 0; e < kv.count; ++e) {
        kv.str_pos.push_back(c.pos());
        uint64_t sat, slen;
        int serr = IFX_GGUF_OK;
        if (!c.string(&sat, &slen, &serr)) return serr;
      }
    } else {
      const int r = skip_value(c, kv.type, 0);
      if (r) return r;
    }
    g->kv_index[kv.key] = g->kvs.size();
    g->kvs.push_back(std::move(kv));
  }

  for (int64_t i = 0; i < n_tensors; ++i) {
    Tensor t{};
    uint64_t at, len;
    int err = IFX_GGUF_OK;
    if (!c.string(&at, &len, &err)) return err;
    t.name.assign(reinterpret_cast<const char *>(g->map + at), len);
    uint32_t nd = 0;
    if (!c.read(&nd)) return IFX_GGUF_TRUNCATED;
    if (nd == 0 || nd > kMaxDims) return IFX_GGUF_BAD_TENSOR;
    t.n_dims = static_cast<int>(nd);
    for (uint32_t d = 0; d < nd; ++d) {
      if (!c.read(&t.shape[d])) return IFX_GGUF_TRUNCATED;
      if (t.shape[d] <= 0) return IFX_GGUF_BAD_TENSOR;
    }
    uint32_t type = 0;
    if (!c.read(&type)) return IFX_GGUF_TRUNCATED;
    if (type > 15) return IFX_GGUF_BAD_TENSOR;
    t.type = static_cast<int>(type);
    if (!c.read(&t.offset)) return IFX_GGUF_TRUNCATED;
    t.bytes = ifx_gguf_tensor_bytes(t.type, t.shape, t.n_dims);
    if (t.bytes == 0) return IFX_GGUF_BAD_TENSOR;
    auto it = g->tensor_index.find(t.name);
    if (it != g->tensor_index.end()) {
      g->tensors[it->second] = std::move(t);  // last definition wins
    } else {
      g->tensor_index[t.name] = static_cast<int64_t>(g->tensors.size());
      g->tensors.push_back(std::move(t));
    }
  }

  g->data_offset = align_up(c.pos(), g->alignment);
  for (const Tensor &t : g->tensors) {
    if (t.offset > g->size || g->data_offset > g->size - t.offset ||
        t.bytes > g->size - g->data_offset - t.offset)
      return IFX_GGUF_BAD_DATA;
  }
  return IFX_GGUF_OK;
}

int check_int_type(uint32_t t) {
  switch (t) {
  case IFX_GGUF_U8: case IFX_GGUF_I8: case IFX_GGUF_U16: case IFX_GGUF_I16:
  case IFX_GGUF_U32: case IFX_GGUF_I32: case IFX_GGUF_U64: case IFX_GGUF_I64:
  case IFX_GGUF_BOOL: return 1;
  default: return 0;
  }
}

}  // namespace

extern "C" {

int ifx_gguf_open(const char *path, ifx_gguf **out) {
  if (!path || !out) return IFX_GGUF_ARGUMENT;
  *out = nullptr;
  auto *g = new ifx_gguf();
  g->fd = open(path, O_RDONLY | O_CLOEXEC);
  struct stat st{};
  if (g->fd < 0 || fstat(g->fd, &st) != 0) {
    delete g;
    return IFX_GGUF_IO;
  }
  g->size = static_cast<uint64_t>(st.st_size);
  if (g->size > 0) {
    void *m = mmap(nullptr, g->size, PROT_READ, MAP_PRIVATE, g->fd, 0);
    if (m == MAP_FAILED) {
      g->size = 0;
      delete g;
      return IFX_GGUF_IO;
    }
    g->map = static_cast<const uint8_t *>(m);
  }
  const int r = parse(g);
  if (r) {
    delete g;
    return r;
  }
  *out = g;
  return IFX_GGUF_OK;
}

void ifx_gguf_close(ifx_gguf *g) { delete g; }

uint32_t ifx_gguf_version(const ifx_gguf *g) { return g ? g->version : 0; }
uint64_t ifx_gguf_alignment(const ifx_gguf *g) { return g ? g->alignment : 0; }
uint64_t ifx_gguf_data_offset(const ifx_gguf *g) { return g ? g->data_offset : 0; }
int64_t ifx_gguf_n_tensors(const ifx_gguf *g) { return g ? static_cast<int64_t>(g->tensors.size()) : 0; }
int64_t ifx_gguf_n_kv(const ifx_gguf *g) { return g ? static_cast<int64_t>(g->kvs.size()) : 0; }

int ifx_gguf_tensor_info(const ifx_gguf *g, int64_t i, ifx_gguf_tensor *out) {
  if (!g || !out) return IFX_GGUF_ARGUMENT;
  if (i < 0 || i >= static_cast<int64_t>(g->tensors.size())) return IFX_GGUF_NOT_FOUND;
  const Tensor &t = g->tensors[static_cast<size_t>(i)];
  out->name = t.name.c_str();
  out->type = t.type;
  out->n_dims = t.n_dims;
  for (int d = 0; d < kMaxDims; ++d) out->shape[d] = d < t.n_dims ? t.shape[d] : 1;
  out->offset = t.offset;
  out->byte_size = t.bytes;
  out->host_data = g->map + g->data_offset + t.offset;
  return IFX_GGUF_OK;
}

int64_t ifx_gguf_find(const ifx_gguf *g, const char *name) {
  if (!g || !name) return -1;
  auto it = g->tensor_index.find(name);
  return it == g->tensor_index.end() ? -1 : it->second;
}

int ifx_gguf_kv_key(const ifx_gguf *g, int64_t i, const char **key, int *value_type) {
  if (!g || !key || !value_type) return IFX_GGUF_ARGUMENT;
  if (i < 0 || i >= static_cast<int64_t>(g->kvs.size())) return IFX_GGUF_NOT_FOUND;
  *key = g->kvs[static_cast<size_t>(i)].key.c_str();
  *value_type = static_cast<int>(g->kvs[static_cast<size_t>(i)].type);
  return IFX_GGUF_OK;
}

int ifx_gguf_get_int(const ifx_gguf *g, const char *key, int64_t *out) {
  if (!g || !out) return IFX_GGUF_ARGUMENT;
  const KV *kv = g->kv(key);
  if (!kv) return IFX_GGUF_NOT_FOUND;
  if (!check_int_type(kv->type)) return IFX_GGUF_WRONG_TYPE;
  const uint8_t *p = g->map + kv->pos;
  switch (kv->type) {
  case IFX_GGUF_U8: case IFX_GGUF_BOOL: *out = p[0]; break;
  case IFX_GGUF_I8: *out = static_cast<int8_t>(p[0]); break;
  case IFX_GGUF_U16: { uint16_t v; std::memcpy(&v, p, 2); *out = v; break; }
  case IFX_GGUF_I16: { int16_t v; std::memcpy(&v, p, 2); *out = v; break; }
  case IFX_GGUF_U32: { uint32_t v; std::memcpy(&v, p, 4); *out = v; break; }
  case IFX_GGUF_I32: { int32_t v; std::memcpy(&v, p, 4); *out = v; break; }
  case IFX_GGUF_U64: {
    uint64_t v;
    std::memcpy(&v, p, 8);
    if (v > static_cast<uint64_t>(INT64_MAX)) return IFX_GGUF_WRONG_TYPE;
    *out = static_cast<int64_t>(v);
    break;
  }
  default: { int64_t v; std::memcpy(&v, p, 8); *out = v; break; }
  }
  return IFX_GGUF_OK;
}

int ifx_gguf_get_float(const ifx_gguf *g, const char *key, double *out) {
  if (!g || !out) return IFX_GGUF_ARGUMENT;
  const KV *kv = g->kv(key);
  if (!kv) return IFX_GGUF_NOT_FOUND;
  const uint8_t *p = g->map + kv->pos;
  if (kv->type == IFX_GGUF_F32) {
    float v;
    std::memcpy(&v, p, 4);
    *out = v;
  } else if (kv->type == IFX_GGUF_F64) {
    std::memcpy(out, p, 8);
  } else {
    return IFX_GGUF_WRONG_TYPE;
  }
  return IFX_GGUF_OK;
}

int ifx_gguf_get_string(const ifx_gguf *g, const char *key, const char **str, uint64_t *len) {
  if (!g || !str || !len) return IFX_GGUF_ARGUMENT;
  const KV *kv = g->kv(key);
  if (!kv) return IFX_GGUF_NOT_FOUND;
  if (kv->type != IFX_GGUF_STRING) return IFX_GGUF_WRONG_TYPE;
  std::memcpy(len, g->map + kv->pos, 8);
  *str = reinterpret_cast<const char *>(g->map + kv->pos + 8);
  return IFX_GGUF_OK;
}

int ifx_gguf_get_array(const ifx_gguf *g, const char *key, int *elem_type, uint64_t *count) {
  if (!g || !elem_type || !count) return IFX_GGUF_ARGUMENT;
  const KV *kv = g->kv(key);
  if (!kv) return IFX_GGUF_NOT_FOUND;
  if (kv->type != IFX_GGUF_ARRAY) return IFX_GGUF_WRONG_TYPE;
  *elem_type = static_cast<int>(kv->elem_type);
  *count = kv->count;
  return IFX_GGUF_OK;
}

int ifx_gguf_get_array_string(const ifx_gguf *g, const char *key, uint64_t idx, const char **str,
                              uint64_t *len) {
  if (!g || !str || !len) return IFX_GGUF_ARGUMENT;
  const KV *kv = g->kv(key);
  if (!kv) return IFX_GGUF_NOT_FOUND;
  if (kv->type != IFX_GGUF_ARRAY || kv->elem_type != IFX_GGUF_STRING) return IFX_GGUF_WRONG_TYPE;
  if (idx >= kv->count) return IFX_GGUF_NOT_FOUND;
  // validated during parsing: a u64 length, then the bytes
  const uint64_t at = kv->str_pos[idx];
  std::memcpy(len, g->map + at, 8);
  *str = reinterpret_cast<const char *>(g->map + at + 8);
  return IFX_GGUF_OK;
}

int ifx_gguf_get_array_data(const ifx_gguf *g, const char *key, const void **data,
                            int *elem_type, uint64_t *count) {
  if (!g || !data || !elem_type || !count) return IFX_GGUF_ARGUMENT;
  const KV *kv = g->kv(key);
  if (!kv) return IFX_GGUF_NOT_FOUND;
  if (kv->type != IFX_GGUF_ARRAY || fixed_size(kv->elem_type) == 0) return IFX_GGUF_WRONG_TYPE;
  *data = g->map + kv->first_elem;
  *elem_type = static_cast<int>(kv->elem_type);
  *count = kv->count;
  return IFX_GGUF_OK;
}

uint64_t ifx_gguf_device_bytes(const ifx_gguf *g, uint64_t align) {
  if (!g || align < 16 || !is_pow2(align)) return 0;
  uint64_t total = 0;
  for (const Tensor &t : g->tensors) total = align_up(total, align) + t.bytes;
  return align_up(total, align);
}

int ifx_gguf_upload(const ifx_gguf *g, void *device, uint64_t device_bytes, uint64_t align,
                    uint64_t *offsets_out, void *stream) {
  if (!g || !device) return IFX_GGUF_ARGUMENT;
  const uint64_t need = ifx_gguf_device_bytes(g, align);
  if (need == 0 && !g->tensors.empty()) return IFX_GGUF_ARGUMENT;
  if (device_bytes < need) return IFX_GGUF_ARGUMENT;
  hipStream_t s = static_cast<hipStream_t>(stream);

  // Pinned double-buffered staging: memcpy from the mapping into one slot
  // while the DMA engine drains the other.
  constexpr uint64_t kChunk = 32ull << 20;
  void *stage[2] = {nullptr, nullptr};
  hipEvent_t done[2] = {nullptr, nullptr};
  bool used[2] = {false, false};
  hipError_t e = hipSuccess;
  for (int i = 0; i < 2 && e == hipSuccess; ++i) {
    e = hipHostMalloc(&stage[i], kChunk, hipHostMallocDefault);
    if (e == hipSuccess) e = hipEventCreateWithFlags(&done[i], hipEventDisableTiming);
  }
  uint64_t dst = 0;
  int slot = 0;
  for (size_t ti = 0; ti < g->tensors.size() && e == hipSuccess; ++ti) {
    const Tensor &t = g->tensors[ti];
    dst = align_up(dst, align);
    if (offsets_out) offsets_out[ti] = dst;
    const uint8_t *src = g->map + g->data_offset + t.offset;
    for (uint64_t done_b = 0; done_b < t.bytes && e == hipSuccess;) {
      const uint64_t n = std::min(kChunk, t.bytes - done_b);
      if (used[slot]) e = hipEventSynchronize(done[slot]);
      if (e != hipSuccess) break;
      std::memcpy(stage[slot], src + done_b, n);
      e = hipMemcpyAsync(static_cast<uint8_t *>(device) + dst + done_b, stage[slot], n,
                         hipMemcpyHostToDevice, s);
      if (e == hipSuccess) e = hipEventRecord(done[slot], s);
      used[slot] = true;
      slot ^= 1;
      done_b += n;
    }
    dst += t.bytes;
  }
  if (e == hipSuccess) e = hipStreamSynchronize(s);
  for (int i = 0; i < 2; ++i) {
    if (done[i]) (void)hipEventDestroy(done[i]);
    if (stage[i]) (void)hipHostFree(stage[i]);
  }
  return e == hipSuccess ? IFX_GGUF_OK : -static_cast<int>(e);
}

uint64_t ifx_gguf_tensor_bytes(int type, const int64_t *shape, int n_dims) {
  if (!shape || n_dims <= 0 || n_dims > kMaxDims) return 0;
  uint64_t n = 1;
  for (int d = 0; d < n_dims; ++d) {
    if (shape[d] <= 0) return 0;
    const uint64_t v = static_cast<uint64_t>(shape[d]);
    if (n > UINT64_MAX / v) return 0;
    n *= v;
  }
  uint64_t be = 0, bb = 0;
  if (!type_block(type, &be, &bb)) return 0;
  const uint64_t blocks = (n + be - 1) / be;  // gguf_util.cpp:548 rounds up
  if (blocks > UINT64_MAX / bb) return 0;
  return blocks * bb;
}

const char *ifx_gguf_type_name(int type) {
  switch (type) {
  case 0: return "f32";
  case 1: return "f16";
  case 2: return "q4_0";
  case 3: return "q4_1";
  case 6: return "q5_0";
  case 7: return "q5_1";
  case 8: return "q8_0";
  case 9: return "q8_1";
  case 10: return "q2_k";
  case 11: return "q3_k";
  case 12: return "q4_k";
  case 13: return "q5_k";
  case 14: return "q6_k";
  case 15: return "q8_k";
  default: return "unknown";
  }
}

int ifx_gguf_parse_name(const char *name, int *layer, char *component, uint64_t component_cap,
                        char *kind, uint64_t kind_cap) {
  if (!name || !layer) return IFX_GGUF_ARGUMENT;
  const std::string s(name);
  std::string comp, knd;
  int l = -1;
  if (s == "tok_emb.weight" || s == "token_embd.weight") {
    comp = "tok_emb";
    knd = "weight";
  } else if (s == "output.weight" || s == "lm_head.weight") {
    l = -2;
    comp = "output";
    knd = "weight";
  } else {
    const size_t d1 = s.find('.');
    const size_t d2 = d1 == std::string::npos ? d1 : s.find('.', d1 + 1);
    if (d1 != std::string::npos && s.compare(0, d1, "blk") == 0 && d2 != std::string::npos) {
      const std::string num = s.substr(d1 + 1, d2 - d1 - 1);
      if (!num.empty() && num.size() < 10 &&
          std::all_of(num.begin(), num.end(), [](char ch) { return ch >= '0' && ch <= '9'; })) {
        l = std::stoi(num);
        const size_t d3 = s.find('.', d2 + 1);
        if (d3 == std::string::npos) {
          comp = s.substr(d2 + 1);
          knd = "weight";
        } else {
          comp = s.substr(d2 + 1, d3 - d2 - 1);
          knd = s.substr(d3 + 1);
        }
      }
    }
  }
  *layer = l;
  auto put = [](const std::string &v, char *dst, uint64_t cap) {
    if (!dst || cap == 0) return;
    const size_t n = std::min<uint64_t>(v.size(), cap - 1);
    std::memcpy(dst, v.data(), n);
    dst[n] = '\0';
  };
  put(comp, component, component_cap);
  put(knd, kind, kind_cap);
  return IFX_GGUF_OK;
}

const char *ifx_gguf_status_string(int status) {
  switch (status) {
  case IFX_GGUF_OK: return "ok";
  case IFX_GGUF_IO: return "cannot open or map the file";
  case IFX_GGUF_BAD_MAGIC: return "not a GGUF file (bad magic)";
  case IFX_GGUF_BAD_VERSION: return "unsupported GGUF version";
  case IFX_GGUF_TRUNCATED: return "file truncated";
  case IFX_GGUF_BAD_KV: return "invalid metadata value";
  case IFX_GGUF_BAD_TENSOR: return "invalid tensor info";
  case IFX_GGUF_BAD_DATA: return "tensor data outside the file";
  case IFX_GGUF_NOT_FOUND: return "not found";
  case IFX_GGUF_WRONG_TYPE: return "metadata value has another type";
  case IFX_GGUF_ARGUMENT: return "bad argument";
  default: return status < 0 ? hipGetErrorString(static_cast<hipError_t>(-status)) : "unknown";
  }
}

}  // extern "C"
