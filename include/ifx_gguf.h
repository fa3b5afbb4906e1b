/*
 * ifx_gguf.h -- C ABI of the GGUF weight loader that feeds the quantized
 * GEMV/GEMM path: GGUF v2/v3 file -> tensor table + metadata -> one device
 * buffer holding every tensor's raw blocks (the layout ifx_qgemm.h reads).
 *
 * Replaces the parsing and upload halves of the reference's GGUFModelLoader
 * (runtime/backends/cuda/native/gguf_model_loader.cpp:284-349 Load,
 * 351-374 ParseHeader, 376-761 ParseKeyValuePairs, 763-848 ParseTensorInfo,
 * 850-901 LoadTensorData, 1005-1047 UploadToGPU) and the helpers of
 * gguf_util.h:97-197 (ReadString, ValidateGGUFHeader, CalcTensorSize,
 * TensorTypeToString, ParseTensorName).
 *
 * Differences by design (same accept/reject decisions, same byte sizes):
 *  - the file is memory-mapped; tensor bytes are never copied into host
 *    vectors (the reference freads every tensor into a std::vector);
 *  - the upload goes into ONE caller-sized device buffer, each tensor at an
 *    `align`-byte boundary (256 by default: whole 128-bit loads and buffer
 *    resources from any tensor base), through a pinned double-buffered
 *    staging ring so the copy runs at DMA speed from pageable file pages;
 *  - every key/value pair is kept (typed getters), not only the keys the
 *    reference's model-info extraction reads.
 *
 * Status codes: 0 = ok; > 0 = the file is not a valid/supported GGUF
 * (enum ifx_gguf_status); < 0 = -(hipError_t) from the upload.
 */
#ifndef IFX_GGUF_H
#define IFX_GGUF_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum ifx_gguf_status {
  IFX_GGUF_OK = 0,
  IFX_GGUF_IO = 10,          /* cannot open / map the file                      */
  IFX_GGUF_BAD_MAGIC = 11,   /* not "GGUF"                                      */
  IFX_GGUF_BAD_VERSION = 12, /* version 0/1 (legacy) or newer than 3            */
  IFX_GGUF_TRUNCATED = 13,   /* a header/metadata/tensor-info read runs past EOF */
  IFX_GGUF_BAD_KV = 14,      /* bad value type, oversize string/array, bad alignment */
  IFX_GGUF_BAD_TENSOR = 15,  /* 0 or > 8 dims, dim <= 0, type id > 15 or without a block size */
  IFX_GGUF_BAD_DATA = 16,    /* tensor bytes lie outside the file              */
  IFX_GGUF_NOT_FOUND = 17,   /* no such key / tensor index                      */
  IFX_GGUF_WRONG_TYPE = 18,  /* key exists with another value type              */
  IFX_GGUF_ARGUMENT = 19     /* null pointer, buffer too small, bad alignment arg */
};

/* GGUF metadata value types (gguf_util.h:30-45). */
enum ifx_gguf_value_type {
  IFX_GGUF_U8 = 0, IFX_GGUF_I8 = 1, IFX_GGUF_U16 = 2, IFX_GGUF_I16 = 3,
  IFX_GGUF_U32 = 4, IFX_GGUF_I32 = 5, IFX_GGUF_F32 = 6, IFX_GGUF_BOOL = 7,
  IFX_GGUF_STRING = 8, IFX_GGUF_ARRAY = 9, IFX_GGUF_U64 = 10, IFX_GGUF_I64 = 11,
  IFX_GGUF_F64 = 12
};

typedef struct ifx_gguf ifx_gguf; /* opaque: a parsed, mapped file */

typedef struct {
  const char *name;      /* NUL-terminated, owned by the ifx_gguf          */
  int type;              /* GGUF tensor type id (gguf_util.h:48-63)        */
  int n_dims;            /* 1..8                                           */
  int64_t shape[8];      /* ne[0] is the innermost (K for a weight matrix) */
  uint64_t offset;       /* byte offset inside the data section            */
  uint64_t byte_size;    /* CalcTensorSize(type, shape)                    */
  const void *host_data; /* into the file mapping (valid until close)      */
} ifx_gguf_tensor;

/* Parse `path` (gguf_model_loader.cpp:284-349 minus the upload). */
int ifx_gguf_open(const char *path, ifx_gguf **out);
void ifx_gguf_close(ifx_gguf *g);

uint32_t ifx_gguf_version(const ifx_gguf *g);
uint64_t ifx_gguf_alignment(const ifx_gguf *g);     /* general.alignment, default 32 */
uint64_t ifx_gguf_data_offset(const ifx_gguf *g);   /* start of the data section     */
int64_t ifx_gguf_n_tensors(const ifx_gguf *g);
int64_t ifx_gguf_n_kv(const ifx_gguf *g);

/* Tensor i in file order (a repeated name keeps the first position and the
 * last definition, as the reference's name map does); ifx_gguf_find returns
 * the index or -1. */
int ifx_gguf_tensor_info(const ifx_gguf *g, int64_t i, ifx_gguf_tensor *out);
int64_t ifx_gguf_find(const ifx_gguf *g, const char *name);

/* Metadata.  get_int accepts every integer type and bool; get_float f32/f64;
 * get_string returns a pointer into the mapping (not NUL-terminated) and
 * its length; get_array the element type and count of an array value, and
 * get_array_string element `idx` of a string array. */
int ifx_gguf_kv_key(const ifx_gguf *g, int64_t i, const char **key, int *value_type);
int ifx_gguf_get_int(const ifx_gguf *g, const char *key, int64_t *out);
int ifx_gguf_get_float(const ifx_gguf *g, const char *key, double *out);
int ifx_gguf_get_string(const ifx_gguf *g, const char *key, const char **str, uint64_t *len);
int ifx_gguf_get_array(const ifx_gguf *g, const char *key, int *elem_type, uint64_t *count);
int ifx_gguf_get_array_string(const ifx_gguf *g, const char *key, uint64_t idx,
                              const char **str, uint64_t *len);
/* Elements of an array of a fixed-size type (integers, floats, bool), in
 * file byte order (little-endian), as a pointer into the mapping. */
int ifx_gguf_get_array_data(const ifx_gguf *g, const char *key, const void **data,
                            int *elem_type, uint64_t *count);

/* Bytes a device buffer needs for every tensor, each starting at a multiple
 * of `align` (a power of two >= 16); 0 if align is invalid. */
uint64_t ifx_gguf_device_bytes(const ifx_gguf *g, uint64_t align);

/* Copy every tensor into `device` (device_bytes >= ifx_gguf_device_bytes)
 * at the aligned offsets, written to offsets_out[n_tensors] when not NULL.
 * Enqueued on `stream`; returns after the last copy has completed (the
 * staging ring is reused), like UploadToGPU's final synchronisation. */
int ifx_gguf_upload(const ifx_gguf *g, void *device, uint64_t device_bytes, uint64_t align,
                    uint64_t *offsets_out, void *stream);

/* gguf_util.cpp:514-577: bytes of a tensor of `type` and shape; 0 = invalid. */
uint64_t ifx_gguf_tensor_bytes(int type, const int64_t *shape, int n_dims);
/* gguf_util.cpp:441-457 ("q4_k", ...; "unknown"). */
const char *ifx_gguf_type_name(int type);
/* gguf_util.cpp:218-268: "blk.N.component.kind" -> layer N (>= 0); token
 * embeddings -> -1, output/lm_head -> -2; other names -> -1 with an empty
 * component.  component/kind are copied NUL-terminated (truncated to cap). */
int ifx_gguf_parse_name(const char *name, int *layer, char *component, uint64_t component_cap,
                        char *kind, uint64_t kind_cap);
const char *ifx_gguf_status_string(int status);

#ifdef __cplusplus
}
#endif

#endif /* IFX_GGUF_H */
