// dequant.hip -- whole-tensor dequantization of raw GGUF blocks on gfx950.
//
// Replaces the reference's dequantize_{q4_k,q5_k,q6_k,q8_0,q8_k} kernels
// (runtime/backends/cuda/native/kernels/dequantization.cu:14-230) and uses
// the element formulas of kernels/quant_common.cuh:100-199:
//   Q4_K  w = d*sc*q - dmin*m      Q6_K  w = d*scale*(q-32)     Q8_0  w = d*q
//   Q5_K  as Q4_K with q = nibble + 16*(bit sb of qh[e])        Q8_K  w = d*q (fp32 d)
// evaluated left to right in IEEE fp32 (this file is compiled with
// -ffp-contract=off), so the values are bit-exact with the CPU restatement.
// The output is fp32, or fp16 (round to nearest even) as the reference
// emits.  It serves verification and callers that want a dense copy; the
// GEMV/GEMM kernels never materialise W.
//
// Mapping: one lane per 8 consecutive outputs, so a wave's stores are
// contiguous (16 bytes per lane for fp16, 32 for fp32); the lane reads the
// 8 codes it needs with one buffer load (unaligned offsets are served) and
// its block's header.
#include "ifx_common.h"

namespace ifx {

// 6-bit scale and min of sub-block sb from the 12 scale bytes as three
// little-endian words (quant_common.cuh:83-94).
__device__ __forceinline__ void scale_min_k4(uint32_t s0, uint32_t s1, uint32_t s2, int sb,
                                             int &sc, int &m) {
  const uint32_t by[12] = {s0 & 0xFF, (s0 >> 8) & 0xFF, (s0 >> 16) & 0xFF, s0 >> 24,
                           s1 & 0xFF, (s1 >> 8) & 0xFF, (s1 >> 16) & 0xFF, s1 >> 24,
                           s2 & 0xFF, (s2 >> 8) & 0xFF, (s2 >> 16) & 0xFF, s2 >> 24};
  if (sb < 4) {
    sc = static_cast<int>(by[sb] & 63);
    m = static_cast<int>(by[sb + 4] & 63);
  } else {
    sc = static_cast<int>((by[sb + 4] & 0xF) | ((by[sb - 4] >> 6) << 4));
    m = static_cast<int>((by[sb + 4] >> 4) | ((by[sb] >> 6) << 4));
  }
}

__device__ __forceinline__ int byte_of(u32x2 v, int i) {
  return static_cast<int>(((i < 4 ? v.x : v.y) >> (8 * (i & 3))) & 0xFFu);
}

// t = index of the 8-output group; element i = 8t .. 8t+7 of the tensor,
// all in one 32-value run of one block.
template <int QT, bool F16>
__global__ __launch_bounds__(256) void k_dequant(const uint8_t *__restrict__ W, uint32_t w_bytes,
                                                 void *__restrict__ out, int64_t ngroups) {
  const rsrc_t Wr = make_rsrc(W, w_bytes);
  const int64_t t = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (t >= ngroups) return;
  float w[8];
  if constexpr (QT == kTypeQ4_K || QT == kTypeQ5_K) {
    constexpr int kB = QT == kTypeQ4_K ? kQ4KBytes : kQ5KBytes;
    const uint32_t blk = static_cast<uint32_t>(t >> 5);
    const int i = static_cast<int>(t & 31) * 8;  // element within the super-block
    const int sb = i >> 5, e = i & 31;
    const uint32_t o = blk * kB;
    const u32x4 hdr = bload<u32x4>(Wr, o, 0);
    const float d = h2f(hdr.x & 0xFFFFu), dmin = h2f(hdr.x >> 16);
    int sc, m;
    scale_min_k4(hdr.y, hdr.z, hdr.w, sb, sc, m);
    const uint32_t qs_off = (QT == kTypeQ4_K ? 16 : 48) + (sb >> 1) * 32 + e;
    const u32x2 qv = bload<u32x2>(Wr, o + qs_off, 0);
    u32x2 hv = {0, 0};
    if constexpr (QT == kTypeQ5_K) hv = bload<u32x2>(Wr, o + 16 + e, 0);
    const int shift = (sb & 1) * 4;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      int q = (byte_of(qv, k) >> shift) & 0xF;
      if constexpr (QT == kTypeQ5_K) q |= ((byte_of(hv, k) >> sb) & 1) << 4;
      w[k] = d * static_cast<float>(sc) * static_cast<float>(q) - dmin * static_cast<float>(m);
    }
  } else if constexpr (QT == kTypeQ8_K) {
    const uint32_t blk = static_cast<uint32_t>(t >> 5);
    const int i = static_cast<int>(t & 31) * 8;
    const uint32_t o = blk * kQ8KBytes;
    const float d = __builtin_bit_cast(float, bload<uint32_t>(Wr, o, 0));
    const u32x2 qv = bload<u32x2>(Wr, o + 4 + i, 0);
#pragma unroll
    for (int k = 0; k < 8; ++k)
      w[k] = d * static_cast<float>(static_cast<int8_t>(byte_of(qv, k)));
  } else if constexpr (QT == kTypeQ6_K) {
    const uint32_t blk = static_cast<uint32_t>(t >> 5);
    const int i = static_cast<int>(t & 31) * 8;
    const int g = i >> 7, sub = (i >> 5) & 3, e = i & 31;
    const uint32_t o = blk * kQ6KBytes;
    const float d = h2f(bload<uint16_t>(Wr, o + 208, 0));
    const u32x2 lv = bload<u32x2>(Wr, o + g * 64 + (sub & 1) * 32 + e, 0);
    const u32x2 hv = bload<u32x2>(Wr, o + 128 + g * 32 + e, 0);
    const uint32_t sc2 = bload<uint16_t>(Wr, o + 192 + g * 8 + sub * 2, 0);  // even offset
    const float sc = static_cast<float>(static_cast<int8_t>(sc2 >> (8 * (e >> 4))));
    const int lshift = (sub >= 2) ? 4 : 0;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const int q = (((byte_of(lv, k) >> lshift) & 0xF) | (((byte_of(hv, k) >> (2 * sub)) & 3) << 4)) - 32;
      w[k] = d * sc * static_cast<float>(q);
    }
  } else {
    const uint32_t blk = static_cast<uint32_t>(t >> 2);
    const int e = static_cast<int>(t & 3) * 8;
    const uint32_t o = blk * kQ8_0Bytes;
    const float d = h2f(bload<uint16_t>(Wr, o, 0));
    const u32x2 qv = bload<u32x2>(Wr, o + 2 + e, 0);
#pragma unroll
    for (int k = 0; k < 8; ++k) w[k] = d * static_cast<float>(static_cast<int8_t>(byte_of(qv, k)));
  }
  if constexpr (F16) {
    // fp32 value first, then fp16 (no fused multiply-convert)
    uint32_t h[4];
#pragma unroll
    for (int k = 0; k < 4; ++k)
      h[k] = f2h_bits(materialize_f32(w[2 * k])) | (f2h_bits(materialize_f32(w[2 * k + 1])) << 16);
    *reinterpret_cast<u32x4 *>(static_cast<uint16_t *>(out) + t * 8) = u32x4{h[0], h[1], h[2], h[3]};
  } else {
    f32x4 *o = reinterpret_cast<f32x4 *>(static_cast<float *>(out) + t * 8);
    o[0] = f32x4{w[0], w[1], w[2], w[3]};
    o[1] = f32x4{w[4], w[5], w[6], w[7]};
  }
}

template <int QT>
static void launch_dq(const uint8_t *W, uint32_t w_bytes, void *out, bool f16, int64_t ngroups,
                      hipStream_t s) {
  const dim3 grid(static_cast<unsigned>((ngroups + 255) / 256));
  if (f16)
    IFX_LAUNCH(k_dequant, (QT, true), grid, dim3(256), 0, s, W, w_bytes, out, ngroups);
  else
    IFX_LAUNCH(k_dequant, (QT, false), grid, dim3(256), 0, s, W, w_bytes, out, ngroups);
}

// n_elems must be a multiple of the block size of qtype and the tensor
// below 4 GiB (checked by the caller).
hipError_t launch_dequantize(int qtype, const void *W, void *out, bool f16, int64_t n_elems,
                             hipStream_t stream) {
  const int64_t ngroups = n_elems / 8;
  if (ngroups == 0) return hipSuccess;
  const uint8_t *w = static_cast<const uint8_t *>(W);
  const int64_t bytes = qtype == kTypeQ8_0 ? n_elems / 32 * kQ8_0Bytes
                        : n_elems / 256 * (qtype == kTypeQ4_K   ? kQ4KBytes
                                           : qtype == kTypeQ5_K ? kQ5KBytes
                                           : qtype == kTypeQ6_K ? kQ6KBytes
                                                                : kQ8KBytes);
  const uint32_t wb = static_cast<uint32_t>(bytes);
  switch (qtype) {
  case kTypeQ4_K: launch_dq<kTypeQ4_K>(w, wb, out, f16, ngroups, stream); break;
  case kTypeQ6_K: launch_dq<kTypeQ6_K>(w, wb, out, f16, ngroups, stream); break;
  case kTypeQ8_0: launch_dq<kTypeQ8_0>(w, wb, out, f16, ngroups, stream); break;
  case kTypeQ5_K: launch_dq<kTypeQ5_K>(w, wb, out, f16, ngroups, stream); break;
  case kTypeQ8_K: launch_dq<kTypeQ8_K>(w, wb, out, f16, ngroups, stream); break;
  default: return hipErrorInvalidValue;
  }
  return last_error();
}

// ---------------------------------------------------------------------------
// Row-split repack (ifx_repack): the fields of each GGUF block of a row move
// to separate 16-byte-aligned sections of the row (layouts in ifx_common.h).
// One thread per (row, block); a load-time operation, so plain byte moves.
// Each row's padding bytes are written as zeros by the row's last block.
// ---------------------------------------------------------------------------
template <int QT>
__global__ __launch_bounds__(256) void k_repack(const uint8_t *__restrict__ W,
                                                uint8_t *__restrict__ out, int64_t n_rows, int K) {
  constexpr int kElems = QT == kTypeQ8_0 ? 32 : 256;
  constexpr int kBytes = QT == kTypeQ8_0 ? kQ8_0Bytes : kQ6KBytes;
  const int nb = K / kElems;
  const int64_t t = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (t >= n_rows * nb) return;
  const int64_t row = t / nb;
  const int b = static_cast<int>(t % nb);
  const uint8_t *src = W + t * kBytes;
  const int rs = row_bytes(QT == kTypeQ8_0 ? kTypeQ8_0R : kTypeQ6_KR, K);
  uint8_t *dst = out + row * rs;
  int end;  // end of the row's data sections
  if constexpr (QT == kTypeQ8_0) {
    for (int i = 0; i < 32; ++i) dst[32 * b + i] = src[2 + i];
    dst[K + 2 * b] = src[0];
    dst[K + 2 * b + 1] = src[1];
    end = K + 2 * nb;
  } else {
    const int qh0 = K / 2, sc0 = qh0 + K / 4, d0 = sc0 + K / 16;
    for (int i = 0; i < 128; ++i) dst[128 * b + i] = src[i];
    for (int i = 0; i < 64; ++i) dst[qh0 + 64 * b + i] = src[128 + i];
    for (int i = 0; i < 16; ++i) dst[sc0 + 16 * b + i] = src[192 + i];
    dst[d0 + 2 * b] = src[208];
    dst[d0 + 2 * b + 1] = src[209];
    end = d0 + 2 * nb;
  }
  if (b == nb - 1)
    for (int i = end; i < rs; ++i) dst[i] = 0;
}

hipError_t launch_repack(int qtype, const void *W, void *out, int64_t n_rows, int K,
                         hipStream_t stream) {
  const int nb = K / (qtype == kTypeQ8_0 ? 32 : 256);
  const int64_t n = n_rows * nb;
  if (n == 0) return hipSuccess;
  const dim3 grid(static_cast<unsigned>((n + 255) / 256));
  const uint8_t *w = static_cast<const uint8_t *>(W);
  uint8_t *o = static_cast<uint8_t *>(out);
  if (qtype == kTypeQ8_0) IFX_LAUNCH(k_repack, (kTypeQ8_0), grid, dim3(256), 0, stream, w, o, n_rows, K);
  else if (qtype == kTypeQ6_K) IFX_LAUNCH(k_repack, (kTypeQ6_K), grid, dim3(256), 0, stream, w, o, n_rows, K);
  else return hipErrorInvalidValue;
  return last_error();
}

// ---------------------------------------------------------------------------
// Tiled repack (ifx_repack_tiled): raw Q4_K / Q6_K rows into the 32-row
// tiles of the batch kernels (layouts in ifx_common.h).  One thread per
// (group, super-block, row of the group); rows past n_rows are zeros.
// ---------------------------------------------------------------------------
template <int QT>
__global__ __launch_bounds__(256) void k_repack_tiled(const uint8_t *__restrict__ W,
                                                      uint8_t *__restrict__ out, int64_t n_rows,
                                                      int K) {
  // bytes of a row's 256 values: one super-block, or eight Q8_0 blocks
  constexpr int kBytes = QT == kTypeQ4_K ? kQ4KBytes : QT == kTypeQ8_0 ? 8 * kQ8_0Bytes : kQ6KBytes;
  constexpr int kTile = kTileRows * kBytes;
  const int nsb = K / 256;
  const int64_t groups = (n_rows + kTileRows - 1) / kTileRows;
  const int64_t t = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (t >= groups * nsb * kTileRows) return;
  const int c = static_cast<int>(t % kTileRows);
  const int64_t gb = t / kTileRows;  // group * nsb + super-block: the tile index
  const int64_t row = (gb / nsb) * kTileRows + c;
  const int b = static_cast<int>(gb % nsb);
  uint8_t *tile = out + gb * kTile;
  uint8_t src[kBytes];
  if (row < n_rows) {
    const uint8_t *p = W + (row * nsb + b) * kBytes;
    for (int i = 0; i < kBytes; ++i) src[i] = p[i];
  } else {
    for (int i = 0; i < kBytes; ++i) src[i] = 0;
  }
  if constexpr (QT == kTypeQ8_0) {
    for (int j = 0; j < 8; ++j) {
      tile[8192 + 16 * c + 2 * j] = src[34 * j];
      tile[8192 + 16 * c + 2 * j + 1] = src[34 * j + 1];
      for (int h = 0; h < 2; ++h)
        for (int i = 0; i < 16; ++i) tile[1024 * j + 512 * h + 16 * c + i] = src[34 * j + 2 + 16 * h + i];
    }
  } else if constexpr (QT == kTypeQ4_K) {
    for (int i = 0; i < 16; ++i) tile[16 * c + i] = src[i];
    for (int p = 0; p < 4; ++p)
      for (int h = 0; h < 2; ++h)
        for (int i = 0; i < 16; ++i) tile[512 + 1024 * p + 512 * h + 16 * c + i] = src[16 + 32 * p + 16 * h + i];
  } else {
    for (int q = 0; q < 4; ++q)
      for (int h = 0; h < 2; ++h)
        for (int i = 0; i < 16; ++i) tile[1024 * q + 512 * h + 16 * c + i] = src[32 * q + 16 * h + i];
    for (int g = 0; g < 2; ++g)
      for (int h = 0; h < 2; ++h)
        for (int i = 0; i < 16; ++i)
          tile[4096 + 1024 * g + 512 * h + 16 * c + i] = src[128 + 32 * g + 16 * h + i];
    for (int i = 0; i < 16; ++i) tile[6144 + 16 * c + i] = src[192 + i];
    tile[6656 + 2 * c] = src[208];
    tile[6656 + 2 * c + 1] = src[209];
  }
}

hipError_t launch_repack_tiled(int qtype, const void *W, void *out, int64_t n_rows, int K,
                               hipStream_t stream) {
  const int64_t n = (n_rows + kTileRows - 1) / kTileRows * (K / 256) * kTileRows;
  if (n == 0) return hipSuccess;
  const dim3 grid(static_cast<unsigned>((n + 255) / 256));
  const uint8_t *w = static_cast<const uint8_t *>(W);
  uint8_t *o = static_cast<uint8_t *>(out);
  if (qtype == kTypeQ4_K) IFX_LAUNCH(k_repack_tiled, (kTypeQ4_K), grid, dim3(256), 0, stream, w, o, n_rows, K);
  else if (qtype == kTypeQ6_K) IFX_LAUNCH(k_repack_tiled, (kTypeQ6_K), grid, dim3(256), 0, stream, w, o, n_rows, K);
  else if (qtype == kTypeQ8_0) IFX_LAUNCH(k_repack_tiled, (kTypeQ8_0), grid, dim3(256), 0, stream, w, o, n_rows, K);
  else return hipErrorInvalidValue;
  return last_error();
}

}  // namespace ifx
