// gemv_dq.hip -- decode-batch GEMV (3 <= M <= 32) on the fp16 matrix cores
// of gfx950: each wave dequantizes its 32 weight rows straight into fp16
// MFMA operands, so the VALU work per weight does not grow with M.
//
// y[m][n] (op)= sum_k W[n][k] * x[m][k], W raw GGUF Q4_K / Q6_K / Q8_0, x
// given as Q8_1 blocks.  The integer-dot kernels (mmvq.hip, mmq_skinny.hip)
// rescale every 32-value block result per output, which is VALU work that
// grows with M (two to three operations per output per block) and at M = 32
// costs as much as the weights take to stream.  Here the weights become fp16
// once, as in the reference's FP16 dequantize path
// (runtime/backends/cuda/native/kernels/quant_common.cuh:100-188):
//   Q4_K  w = fp16(d*sc) * q - fp16(dmin*m)
//   Q6_K  w = fp16(d*sc) * (q - 32)
//   Q8_0  w = fp16(d) * q
// and x = fp16(d_a) * q_a; v_mfma_f32_32x32x16_f16 accumulates in fp32.
// The fp16 rounding of w and x (relative 2^-11) stays far inside the
// contract's 1e-3 * ||y_row|| tolerance at every decode shape.
//
// Mapping: MFMA A operand = 32 batch rows (rows >= M read a zero row),
// B operand = 32 weight rows; lane l supplies row / column l % 32 for the
// 8-value K group l / 32 and receives column n = l % 32, rows
// 8*(i/4) + 4*(l/32) + (i%4).  Both lanes of a weight row (l, l + 32) load
// 16-byte pieces of it side by side (32 contiguous bytes per row and load
// instruction): Q4_K 16 B of each 32-byte qs chunk plus the header; the
// eight values an MFMA takes from a lane are 16*h + (0..7 or 8..15) of one
// sub-block, in the order (0, 2, 1, 3) of each group of four that the
// packed conversion produces; the activations are staged in that order.
//
// Workgroup: 4 waves = 128 weight rows over a range of super-blocks (K split
// over gridDim.y with fp32 atomics when the rows alone cannot fill the
// chip).  Per super-block the workgroup converts the batch rows' Q8_1
// blocks into a double-buffered LDS stage (M x 256 fp16) that all four
// waves read; the next super-block's weight bytes are loaded while the
// current one is computed.
#include "ifx_common.h"
#include "ifx_q8_1.h"

#include <stdlib.h>

#include <algorithm>
#include <type_traits>

namespace ifx {

namespace {

typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef _Float16 h8 __attribute__((ext_vector_type(8)));

constexpr int kWaves = 4;
constexpr int kRowsPerWg = 32 * kWaves;
constexpr int kMaxM = 32;
constexpr int kLdsBytes = 65536;  // activation stage: two workgroups per CU
constexpr uint32_t kMagic = 0x64006400u;  // fp16 1024.0 in both halves

struct DqSeg {
  const uint8_t *W;
  void *Y;
  const void *bias;
  int N;
  int blk_begin;
};
struct DqArgs {
  DqSeg seg[3];
  int nseg;
  const uint8_t *A;
  int M, K, mode, sb_per;
  SplitWs ws;  // ordered split: counters per row group, 16 KB slot per (group, split)
  // fused gate/up/SiLU (SW): seg[0] gate, seg[1] up; h = silu(g) * u to H
  // (fp32, or fp16 with h_f16; or none) and its Q8_1 blocks to Q (or none)
  void *H;
  uint8_t *Q;
  int h_f16;
};

__device__ __forceinline__ h2 as_h2(uint32_t u) { return __builtin_bit_cast(h2, u); }
__device__ __forceinline__ uint32_t as_u32(h2 h) { return __builtin_bit_cast(uint32_t, h); }
__device__ __forceinline__ h2 splat(float f) {
  const _Float16 h = static_cast<_Float16>(f);
  return h2{h, h};
}

// Signed byte codes (four per word) times d -> fp16 pairs of values (0, 2)
// and (1, 3): (0x6400 | (q ^ 0x80)) - 1152 = q exactly, one rounding.
__device__ __forceinline__ void i8x4_to_h(uint32_t x, h2 d, uint32_t &p02, uint32_t &p13) {
  const uint32_t mg = vreg(kMagic);
  x ^= 0x80808080u;
  const h2 off = splat(-1152.0f);
  p02 = as_u32((as_h2((x & 0x00FF00FFu) | mg) + off) * d);
  p13 = as_u32((as_h2(((x >> 8) & 0x00FF00FFu) | mg) + off) * d);
}

// Byte codes v (< 1024, four per word) -> fp16 pairs (v + bias) * d - mn of
// values (0, 2) and (1, 3).
__device__ __forceinline__ void u8x4_to_h(uint32_t x, h2 bias, h2 d, h2 mn, uint32_t &p02,
                                          uint32_t &p13) {
  const uint32_t mg = vreg(kMagic);
  const h2 a = as_h2((x & 0x00FF00FFu) | mg) + bias;
  const h2 b = as_h2(((x >> 8) & 0x00FF00FFu) | mg) + bias;
  p02 = as_u32(__builtin_elementwise_fma(a, d, -mn));
  p13 = as_u32(__builtin_elementwise_fma(b, d, -mn));
}

// Nibble codes (HI = 0: low, 1: high nibbles) of two words of packed 4-bit
// codes -> one 8-value operand q * d - mn.  Low nibbles sit in mantissa
// bits 0..3 under the magic 1024 (ulp 1): 1024 + q; high nibbles stay in
// bits 4..7, under the magic 64 (0x5400, ulp 1/16) also exactly 64 + q; so
// one shift per word serves both, and each pair is one and-or.
template <int HI>
__device__ __forceinline__ h8 op_q4(uint32_t x0, uint32_t x1, h2 d, h2 mn) {
  constexpr uint32_t msk = HI ? 0x00F000F0u : 0x000F000Fu;
  const uint32_t mg = vreg(HI ? 0x54005400u : kMagic);
  const h2 bias = splat(HI ? -64.0f : -1024.0f);
  const uint32_t w[4] = {(x0 & msk) | mg, ((x0 >> 8) & msk) | mg, (x1 & msk) | mg,
                         ((x1 >> 8) & msk) | mg};
  uint32_t o[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) o[i] = as_u32(__builtin_elementwise_fma(as_h2(w[i]) + bias, d, -mn));
  return __builtin_bit_cast(h8, u32x4{o[0], o[1], o[2], o[3]});
}

// Two words of byte codes -> one 8-value operand.
__device__ __forceinline__ h8 op_u8(uint32_t x0, uint32_t x1, h2 bias, h2 d, h2 mn) {
  uint32_t o[4];
  u8x4_to_h(x0, bias, d, mn, o[0], o[1]);
  u8x4_to_h(x1, bias, d, mn, o[2], o[3]);
  return __builtin_bit_cast(h8, u32x4{o[0], o[1], o[2], o[3]});
}
__device__ __forceinline__ h8 op_i8(uint32_t x0, uint32_t x1, h2 d) {
  uint32_t o[4];
  i8x4_to_h(x0, d, o[0], o[1]);
  i8x4_to_h(x1, d, o[2], o[3]);
  return __builtin_bit_cast(h8, u32x4{o[0], o[1], o[2], o[3]});
}

// One super-block of a lane's weight row in registers.
template <int QT>
struct RawW;
template <>
struct RawW<kTypeQ4_K> {  // header, qs bytes 32p + 16h .. +15 for p = 0..3
  u32x4 hdr, qs[4];
};
template <>
struct RawW<kTypeQ6_K> {  // ql bytes 32c + 16h .. (c = 0..3), qh 32g + 16h .., scales, d
  u32x4 ql[4], qh[2], sc;
  uint32_t d;
};
template <>
struct RawW<kTypeQ8_0> {  // codes 16h .. 16h+15 and d of the 8 blocks
  u32x4 q[8];
  uint32_t d[8];
};

// TL: the tiled layout (ifx_common.h); row_off = the first tile of the
// lane's 32-row group, c = lane % 32.
template <int QT, bool TL = false>
__device__ __forceinline__ void fetch_w(RawW<QT> &r, rsrc_t Wr, uint32_t row_off, int sb, int h,
                                        int c = 0) {
  if constexpr (TL && QT == kTypeQ8_0) {
    const uint32_t o = row_off + sb * (kTileRows * 8 * kQ8_0Bytes) + 16 * c;
#pragma unroll
    for (int b = 0; b < 8; ++b) r.q[b] = wload<u32x4>(Wr, o + 1024 * b + 512 * h, 0);
    const u32x4 dd = wload<u32x4>(Wr, o + 8192, 0);
    const uint32_t dw[4] = {dd.x, dd.y, dd.z, dd.w};
#pragma unroll
    for (int b = 0; b < 8; ++b) r.d[b] = (dw[b >> 1] >> (16 * (b & 1))) & 0xFFFFu;
  } else if constexpr (TL && QT == kTypeQ4_K) {
    const uint32_t o = row_off + sb * (kTileRows * kQ4KBytes) + 16 * c;
    r.hdr = wload<u32x4>(Wr, o, 0);
#pragma unroll
    for (int p = 0; p < 4; ++p) r.qs[p] = wload<u32x4>(Wr, o + 512 + 1024 * p + 512 * h, 0);
  } else if constexpr (TL) {
    const uint32_t t = row_off + sb * (kTileRows * kQ6KBytes), o = t + 16 * c;
#pragma unroll
    for (int i = 0; i < 4; ++i) r.ql[i] = wload<u32x4>(Wr, o + 1024 * i + 512 * h, 0);
#pragma unroll
    for (int g = 0; g < 2; ++g) r.qh[g] = wload<u32x4>(Wr, o + 4096 + 1024 * g + 512 * h, 0);
    r.sc = wload<u32x4>(Wr, o + 6144, 0);
    r.d = wload<uint16_t>(Wr, t + 6656 + 2 * c, 0);
  } else if constexpr (QT == kTypeQ4_K) {
    const uint32_t o = row_off + sb * kQ4KBytes;
    r.hdr = wload<u32x4>(Wr, o, 0);
#pragma unroll
    for (int p = 0; p < 4; ++p) r.qs[p] = wload<u32x4>(Wr, o + 16 + 32 * p + 16 * h, 0);
  } else if constexpr (QT == kTypeQ6_K) {
    const uint32_t o = row_off + sb * kQ6KBytes;
#pragma unroll
    for (int c = 0; c < 4; ++c) r.ql[c] = wload<u32x4>(Wr, o + 32 * c + 16 * h, 0);
#pragma unroll
    for (int g = 0; g < 2; ++g) r.qh[g] = wload<u32x4>(Wr, o + 128 + 32 * g + 16 * h, 0);
    r.sc = wload<u32x4>(Wr, o + 192, 0);
    r.d = wload<uint16_t>(Wr, o + 208, 0);
  } else {
    const uint32_t o = row_off + sb * 8 * kQ8_0Bytes;
#pragma unroll
    for (int b = 0; b < 8; ++b) {
      r.d[b] = wload<uint16_t>(Wr, o + b * kQ8_0Bytes, 0);
      r.q[b] = wload<u32x4>(Wr, o + b * kQ8_0Bytes + 2 + 16 * h, 0);
    }
  }
}

// Activation operand: 8 halves of the staged row at value offset `v` of the
// super-block.
__device__ __forceinline__ h8 act(const _Float16 *row, int v) {
  return *reinterpret_cast<const h8 *>(row + v);
}

__device__ __forceinline__ f32x16 mfma(h8 a, h8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

// 16 MFMAs of one super-block into acc0 / acc1 (two chains).
template <int QT>
__device__ __forceinline__ void compute(const RawW<QT> &r, const _Float16 *sa, int h,
                                        f32x16 &acc0, f32x16 &acc1) {
  const int e0 = 16 * h;
  if constexpr (QT == kTypeQ4_K) {
    // get_scale_min_k4 (quant_common.cuh:83-94), all eight sub-blocks
    const float d = h2f(r.hdr.x & 0xFFFFu), dmin = h2f(r.hdr.x >> 16);
    const uint32_t S0 = r.hdr.y, S1 = r.hdr.z, S2 = r.hdr.w;
    const uint32_t sc_lo = S0 & 0x3F3F3F3Fu, m_lo = S1 & 0x3F3F3F3Fu;
    const uint32_t sc_hi = (S2 & 0x0F0F0F0Fu) | ((S0 >> 2) & 0x30303030u);
    const uint32_t m_hi = ((S2 >> 4) & 0x0F0F0F0Fu) | ((S1 >> 2) & 0x30303030u);
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      const uint32_t scw = p < 2 ? sc_lo : sc_hi, mw = p < 2 ? m_lo : m_hi;
      const int sh = 16 * (p & 1);
      const h2 d0 = splat(d * static_cast<float>((scw >> sh) & 0xFFu));
      const h2 d1 = splat(d * static_cast<float>((scw >> (sh + 8)) & 0xFFu));
      const h2 n0 = splat(dmin * static_cast<float>((mw >> sh) & 0xFFu));
      const h2 n1 = splat(dmin * static_cast<float>((mw >> (sh + 8)) & 0xFFu));
      const u32x4 q = r.qs[p];
      const int b0 = 64 * p + e0, b1 = 64 * p + 32 + e0;  // value offsets of the two sub-blocks
      acc0 = mfma(act(sa, b0), op_q4<0>(q.x, q.y, d0, n0), acc0);
      acc1 = mfma(act(sa, b0 + 8), op_q4<0>(q.z, q.w, d0, n0), acc1);
      acc0 = mfma(act(sa, b1), op_q4<1>(q.x, q.y, d1, n1), acc0);
      acc1 = mfma(act(sa, b1 + 8), op_q4<1>(q.z, q.w, d1, n1), acc1);
    }
  } else if constexpr (QT == kTypeQ6_K) {
    // dequant_q6k_element (quant_common.cuh:161-177): chunk c = (g, hf)
    // holds sub-blocks hf (low nibbles, qh bits 2hf..) and hf + 2 (high
    // nibbles, qh bits 2hf + 4 ..) of 128-value half g; the 16 values of a
    // lane share scale g*8 + 2*sub + h.
    const float d = h2f(r.d);
    const uint32_t scb[4] = {r.sc.x, r.sc.y, r.sc.z, r.sc.w};
    const h2 bias = splat(-1056.0f), zero = splat(0.0f);
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int g = c >> 1, hf = c & 1;
      const int ilo = g * 8 + 2 * hf + h, ihi = g * 8 + 2 * (hf + 2) + h;
      const float slo = static_cast<float>(static_cast<int8_t>((scb[ilo >> 2] >> (8 * (ilo & 3))) & 0xFFu));
      const float shi = static_cast<float>(static_cast<int8_t>((scb[ihi >> 2] >> (8 * (ihi & 3))) & 0xFFu));
      const h2 dl = splat(d * slo), dh = splat(d * shi);
      const u32x4 ql = r.ql[c];
      u32x4 y = r.qh[g];
      y = u32x4{y.x >> (2 * hf), y.y >> (2 * hf), y.z >> (2 * hf), y.w >> (2 * hf)};
      const uint32_t lo[4] = {(ql.x & 0x0F0F0F0Fu) | ((y.x << 4) & 0x30303030u),
                              (ql.y & 0x0F0F0F0Fu) | ((y.y << 4) & 0x30303030u),
                              (ql.z & 0x0F0F0F0Fu) | ((y.z << 4) & 0x30303030u),
                              (ql.w & 0x0F0F0F0Fu) | ((y.w << 4) & 0x30303030u)};
      const uint32_t hi[4] = {((ql.x >> 4) & 0x0F0F0F0Fu) | (y.x & 0x30303030u),
                              ((ql.y >> 4) & 0x0F0F0F0Fu) | (y.y & 0x30303030u),
                              ((ql.z >> 4) & 0x0F0F0F0Fu) | (y.z & 0x30303030u),
                              ((ql.w >> 4) & 0x0F0F0F0Fu) | (y.w & 0x30303030u)};
      const int blo = g * 128 + hf * 32 + e0, bhi = g * 128 + (hf + 2) * 32 + e0;
      acc0 = mfma(act(sa, blo), op_u8(lo[0], lo[1], bias, dl, zero), acc0);
      acc1 = mfma(act(sa, blo + 8), op_u8(lo[2], lo[3], bias, dl, zero), acc1);
      acc0 = mfma(act(sa, bhi), op_u8(hi[0], hi[1], bias, dh, zero), acc0);
      acc1 = mfma(act(sa, bhi + 8), op_u8(hi[2], hi[3], bias, dh, zero), acc1);
    }
  } else {
    // dequant_q8_0_element (quant_common.cuh:185-188)
#pragma unroll
    for (int b = 0; b < 8; ++b) {
      const h2 d = splat(h2f(r.d[b]));
      const u32x4 q = r.q[b];
      const int v = 32 * b + e0;
      if (b & 1) {
        acc1 = mfma(act(sa, v), op_i8(q.x, q.y, d), acc1);
        acc1 = mfma(act(sa, v + 8), op_i8(q.z, q.w, d), acc1);
      } else {
        acc0 = mfma(act(sa, v), op_i8(q.x, q.y, d), acc0);
        acc0 = mfma(act(sa, v + 8), op_i8(q.z, q.w, d), acc0);
      }
    }
  }
}

// Stage the activations of super-blocks [sb0, sb0 + cnt) as fp16: row m at
// sa + m * pitch, values in the order (0, 2, 1, 3) of each group of four.
// Up to 4 Q8_1 blocks per thread.  stage_a_load issues the loads with no
// branch around them (items past the end re-read the last one, unused), so
// that the weight loads issued after it do not hold them up (a wave's loads
// complete in issue order); stage_a_store converts and stores.
struct StageA {
  uint32_t ds[4];
  u32x4 q0[4], q1[4];
};

__device__ __forceinline__ void stage_a_load(StageA &st, rsrc_t Ar, uint32_t a_row, int M, int sb0,
                                             int cnt, int tid) {
  const int items = M * 8 * cnt;
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int it = min(tid + 256 * u, items - 1);
    const int m = it / (8 * cnt), j = it - m * 8 * cnt;
    const uint32_t o = m * a_row + (sb0 * 8 + j) * kQ8_1Bytes;
    st.ds[u] = bload<uint32_t>(Ar, o, 0);
    st.q0[u] = bload<u32x4>(Ar, o + 4, 0);
    st.q1[u] = bload<u32x4>(Ar, o + 20, 0);
  }
}

__device__ __forceinline__ void stage_a_store(const StageA &st, _Float16 *sa, int pitch, int M,
                                              int cnt, int tid) {
  const int items = M * 8 * cnt;
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int it = tid + 256 * u;
    if (it < items) {
      const int m = it / (8 * cnt), j = it - m * 8 * cnt;
      const h2 d = splat(h2f(st.ds[u] & 0xFFFFu));
      u32x4 *dst = reinterpret_cast<u32x4 *>(sa + m * pitch + 32 * j);
      const uint32_t in[8] = {st.q0[u].x, st.q0[u].y, st.q0[u].z, st.q0[u].w,
                              st.q1[u].x, st.q1[u].y, st.q1[u].z, st.q1[u].w};
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        uint32_t o[4];
        i8x4_to_h(in[2 * k], d, o[0], o[1]);
        i8x4_to_h(in[2 * k + 1], d, o[2], o[3]);
        dst[k] = u32x4{o[0], o[1], o[2], o[3]};
      }
    }
  }
}

}  // namespace

// grid: x = row groups of 128 (all projections), y = super-block splits.
// Dynamic LDS: (M + 1) rows of pitch = sb_per * 256 + 8 halves (row M zero).
// SPLIT: 0 one workgroup per row group; 1 K split, fp32 atomics into Y
// (zeroed first in store / bias mode); 2 K split, ordered reduction through
// args.ws (split_arrive_last).
// SW: fused gate/up/SiLU.  A workgroup owns 64 outputs: waves 0-1 their
// gate rows, waves 2-3 the same up rows, each row summed exactly as the
// grouped launch with the same K split sums it; after the (ordered)
// reduction the workgroup forms h = silu(g) * u and its Q8_1 blocks with the
// SiLU producer's arithmetic (8 lanes per block), so h and the blocks equal
// grouped GEMV + silu_mul_quantize bit for bit.
template <int QT, bool F16OUT, int SPLIT, bool TL = false, bool SW = false>
__global__ __launch_bounds__(64 * kWaves, 2) void k_gemv_dq(const DqArgs args) {
  extern __shared__ __attribute__((aligned(16))) _Float16 lds[];
  const int bx = blockIdx.x;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: scalar descriptors
  const int si = SW ? wave >> 1  // waves 0-1 gate, 2-3 up
                 : (args.nseg > 2 && bx >= args.seg[2].blk_begin) ? 2
                 : (args.nseg > 1 && bx >= args.seg[1].blk_begin) ? 1 : 0;
  const DqSeg &sg = args.seg[si];
  const int l32 = lane & 31, h = lane >> 5;
  const int M = args.M, K = args.K, N = sg.N;
  const int nsb = K >> 8;
  const int sb_begin = blockIdx.y * args.sb_per;
  const int cnt = min(nsb, sb_begin + args.sb_per) - sb_begin;
  const int pitch = args.sb_per * 256 + 8;  // halves; 4 dwords mod 64 banks

  const uint32_t a_row = static_cast<uint32_t>(K >> 5) * kQ8_1Bytes;
  const uint32_t w_row = static_cast<uint32_t>(
      QT == kTypeQ8_0 ? (K >> 5) * kQ8_0Bytes : (K >> 8) * (QT == kTypeQ4_K ? kQ4KBytes : kQ6KBytes));
  const rsrc_t Wr = make_rsrc(sg.W, w_row * static_cast<uint32_t>(TL ? (N + 31) & ~31 : N));
  const rsrc_t Ar = make_rsrc(args.A, a_row * static_cast<uint32_t>(M));
  const int n = SW ? bx * 64 + (wave & 1) * 32 + l32
                   : (bx - sg.blk_begin) * kRowsPerWg + wave * 32 + l32;
  // tiled: the group's first tile (group-major tiles of 32 rows x 1 super-block)
  const uint32_t row_off = TL ? static_cast<uint32_t>(n >> 5) * 32 * w_row
                              : static_cast<uint32_t>(min(n, N - 1)) * w_row;
  // batch rows past M read the zero row M
  const _Float16 *arow = lds + (l32 < M ? l32 : M) * pitch;

  f32x16 acc0, acc1;
#pragma unroll
  for (int i = 0; i < 16; ++i) acc0[i] = acc1[i] = 0.0f;

  // Three super-blocks of weights in flight per wave (register ring), the
  // first two issued right after the activation stage's loads, so that the
  // stage (small, cache-resident) completes without waiting behind them.
  StageA st;
  stage_a_load(st, Ar, a_row, M, sb_begin, cnt, tid);
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_sched_barrier(0);
  RawW<QT> w0, w1, w2;
  fetch_w<QT, TL>(w0, Wr, row_off, sb_begin, h, l32);  // cnt >= 1
  fetch_w<QT, TL>(w1, Wr, row_off, sb_begin + min(1, cnt - 1), h, l32);
  for (int i = tid; i < pitch / 8; i += 64 * kWaves)
    reinterpret_cast<u32x4 *>(lds + M * pitch)[i] = u32x4{0, 0, 0, 0};
  stage_a_store(st, lds, pitch, M, cnt, tid);
  __syncthreads();

  auto step = [&](const RawW<QT> &cur, RawW<QT> &fut, int i) {
    if (i + 2 < cnt) fetch_w<QT, TL>(fut, Wr, row_off, sb_begin + i + 2, h, l32);
    compute<QT>(cur, arow + 256 * i, h, acc0, acc1);
  };
  for (int i = 0; i < cnt; i += 3) {
    step(w0, w2, i);
    if (i + 1 < cnt) step(w1, w0, i + 1);
    if (i + 2 < cnt) step(w2, w1, i + 2);
  }

  // lane holds column n and batch rows 8*(i/4) + 4*h + (i%4)
  float yv[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) yv[i] = acc0[i] + acc1[i];
  float base[16];  // SPLIT == 2, accumulate mode: Y before this launch
  if constexpr (SPLIT == 2) {
    const int ks = gridDim.y;
    // the accumulate base, requested before the arrival so that its latency
    // overlaps it (only the last workgroup uses it; nothing in this launch
    // writes Y before that workgroup's epilogue)
    const int nc = min(n, N - 1);
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int m = 8 * (i >> 2) + 4 * h + (i & 3);
      base[i] = (!F16OUT && args.mode == 1 && m < M)
                    ? static_cast<const float *>(sg.Y)[static_cast<int64_t>(m) * N + nc] : 0.0f;
    }
    constexpr int kSlot = 64 * 16;  // floats per wave and split
    float *mine = args.ws.part + (static_cast<int64_t>(bx) * ks + blockIdx.y) * kWaves * kSlot +
                  wave * kSlot + lane;
#pragma unroll
    for (int i = 0; i < 16; ++i)
      if (8 * (i >> 2) + 4 * h + (i & 3) < M) st_dev(mine + 64 * i, yv[i]);
    wait_own_memory();
    if (!split_arrive_last(args.ws.cnt + bx, ks)) return;
    // all slots, this workgroup's included, in split order; four slots'
    // loads in flight at a time (rows past M were not stored and are unused)
    const float *slot0 = args.ws.part + static_cast<int64_t>(bx) * ks * kWaves * kSlot + wave * kSlot + lane;
    float t[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) t[i] = 0.0f;
    for (int sp0 = 0; sp0 < ks; sp0 += 4) {
      float v[4][16];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float *src = slot0 + min(sp0 + j, ks - 1) * kWaves * kSlot;
#pragma unroll
        for (int i = 0; i < 16; ++i) v[j][i] = ld_dev(src + 64 * i);
      }
#pragma unroll
      for (int j = 0; j < 4; ++j)
        if (sp0 + j < ks) {
#pragma unroll
          for (int i = 0; i < 16; ++i) t[i] += v[j][i];
        }
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) yv[i] = t[i];
    split_reset(args.ws.cnt + bx);
  }
  if constexpr (SW) {
    // gate / up sums of the 64 outputs -> LDS [projection][batch row][64]
    // (the activation stage is no longer read: every wave has passed a
    // barrier after its last super-block)
    if constexpr (SPLIT != 2) __syncthreads();
    float *gu = reinterpret_cast<float *>(lds);
    const int proj = wave >> 1, col = (wave & 1) * 32 + l32;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int m = 8 * (i >> 2) + 4 * h + (i & 3);
      if (m < M) gu[(proj * kMaxM + m) * 64 + col] = yv[i];
    }
    __syncthreads();
    // 8 lanes per Q8_1 block (4 outputs each), two blocks per batch row;
    // whole 8-lane groups stay active together
    const int n0 = bx * 64;
    for (int it = tid; it < M * 16; it += 64 * kWaves) {
      const int blk = it >> 3, l = it & 7, m = blk >> 1, b = blk & 1;
      const int o = n0 + 32 * b + 4 * l;
      if (n0 + 32 * b >= N) continue;
      const f32x4 g4 = *reinterpret_cast<const f32x4 *>(&gu[m * 64 + 32 * b + 4 * l]);
      const f32x4 u4 = *reinterpret_cast<const f32x4 *>(&gu[(kMaxM + m) * 64 + 32 * b + 4 * l]);
      const f32x4 hv = silu_mul4(g4, u4);
      const int64_t oh = static_cast<int64_t>(m) * N + o;
      if (args.H) {
        if (args.h_f16) {
          const u32x2 hh = {f2h_bits(hv.x) | (f2h_bits(hv.y) << 16),
                            f2h_bits(hv.z) | (f2h_bits(hv.w) << 16)};
          *reinterpret_cast<u32x2 *>(static_cast<uint16_t *>(args.H) + oh) = hh;
        } else {
          *reinterpret_cast<f32x4 *>(static_cast<float *>(args.H) + oh) = hv;
        }
      }
      if (args.Q)
        quantize4_store(hv.x, hv.y, hv.z, hv.w,
                        args.Q + (static_cast<int64_t>(m) * (N >> 5) + (o >> 5)) * kQ8_1Bytes, l);
    }
    return;
  }
  if (n >= N) return;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int m = 8 * (i >> 2) + 4 * h + (i & 3);
    if (m >= M) continue;
    const int64_t o = static_cast<int64_t>(m) * N + n;
    float y = yv[i];
    if constexpr (SPLIT == 1) {
      if (args.mode == 2 && blockIdx.y == 0) y += static_cast<const float *>(sg.bias)[n];
      atomicAdd(static_cast<float *>(sg.Y) + o, y);
    } else if constexpr (F16OUT) {
      uint16_t *Yh = static_cast<uint16_t *>(sg.Y);
      if (args.mode == 1) y += h2f(Yh[o]);
      else if (args.mode == 2) y += h2f(static_cast<const uint16_t *>(sg.bias)[n]);
      Yh[o] = static_cast<uint16_t>(f2h_bits(y));
    } else {
      float *Yf = static_cast<float *>(sg.Y);
      if (args.mode == 1) y += SPLIT == 2 ? base[i] : Yf[o];
      else if (args.mode == 2) y += static_cast<const float *>(sg.bias)[n];
      Yf[o] = y;
    }
  }
}

namespace {

// Rolling-stage form without a K split, for launches wide enough to fill
// the chip with one workgroup per 128-row group (k_gemv_dqr): each workgroup
// walks the whole K of its rows, so the sums need no cross-workgroup
// reduction (no partial-sum traffic, no zero fill, the same bits every run).
// The activations pass through two LDS stages of C super-blocks: the next
// step's Q8_1 loads are issued right after a step's barrier, ahead of that
// step's weight loads, and converted into the idle stage after the step's
// units, so waiting for them waits only for weights the step itself uses
// (a wave's loads complete in issue order).  WV = 8: two waves per row
// slice (one per half of the SIMDs' wave slots), taking alternate
// super-blocks; their sums meet in LDS at the end.  Each wave keeps D of
// its super-blocks in flight across steps.
template <int C, int NT>
struct StageR {
  static constexpr int kSlots = 1024 / NT;  // M * 8 * C <= 1024 Q8_1 blocks
  uint32_t ds[kSlots];
  u32x4 q0[kSlots], q1[kSlots];
};

// Loads of step s (super-blocks s*C .. s*C + C - 1; past the end the last
// one is re-read: finite values that meet zero weights).
template <int C, int NT>
__device__ __forceinline__ void stage_r_load(StageR<C, NT> &st, rsrc_t Ar, uint32_t a_row, int M,
                                             int step, int nsb, int tid) {
  const int items = M * 8 * C;
#pragma unroll
  for (int u = 0; u < StageR<C, NT>::kSlots; ++u) {
    const int it = min(tid + NT * u, items - 1);
    const int m = it / (8 * C), j = it - m * (8 * C);
    const int sb = min(step * C + (j >> 3), nsb - 1);
    const uint32_t o = m * a_row + (sb * 8 + (j & 7)) * kQ8_1Bytes;
    st.ds[u] = bload<uint32_t>(Ar, o, 0);
    st.q0[u] = bload<u32x4>(Ar, o + 4, 0);
    st.q1[u] = bload<u32x4>(Ar, o + 20, 0);
  }
}

template <int C, int NT>
__device__ __forceinline__ void stage_r_store(const StageR<C, NT> &st, _Float16 *sa, int pitch,
                                              int M, int tid) {
  const int items = M * 8 * C;
#pragma unroll
  for (int u = 0; u < StageR<C, NT>::kSlots; ++u) {
    const int it = tid + NT * u;
    if (it < items) {
      const int m = it / (8 * C), j = it - m * (8 * C);
      const h2 d = splat(h2f(st.ds[u] & 0xFFFFu));
      u32x4 *dst = reinterpret_cast<u32x4 *>(sa + m * pitch + 32 * j);
      const uint32_t in[8] = {st.q0[u].x, st.q0[u].y, st.q0[u].z, st.q0[u].w,
                              st.q1[u].x, st.q1[u].y, st.q1[u].z, st.q1[u].w};
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        uint32_t o[4];
        i8x4_to_h(in[2 * k], d, o[0], o[1]);
        i8x4_to_h(in[2 * k + 1], d, o[2], o[3]);
        dst[k] = u32x4{o[0], o[1], o[2], o[3]};
      }
    }
  }
}

}  // namespace

// grid: one workgroup per 128-row group (all projections; SW: 64 outputs,
// row slices 0-1 gate and 2-3 up); 64 * WV threads.  Dynamic LDS: two
// stages of (M + 1) rows of pitch C * 256 + 8 halves (row M zero).
template <int QT, bool F16OUT, bool TL, bool SW, int C, int D, int WV>
__global__ __launch_bounds__(64 * WV, 1) void k_gemv_dqr(const DqArgs args) {
  constexpr int NT = 64 * WV, kHalves = WV / 4, Cw = C / kHalves;
  static_assert((WV == 4 || WV == 8) && C % kHalves == 0, "row slices");
  static_assert(D == Cw || D == 2 * Cw, "ring and stage steps");
  [[maybe_unused]] constexpr int kStampBase = 0;
  IFX_STAMP(0);
  extern __shared__ __attribute__((aligned(16))) _Float16 lds[];
  const int bx = blockIdx.x;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: scalar descriptors
  const int rw = wave & 3, half = wave >> 2;  // row slice; which super-blocks (WV = 8)
  const int si = SW ? rw >> 1
                 : (args.nseg > 2 && bx >= args.seg[2].blk_begin) ? 2
                 : (args.nseg > 1 && bx >= args.seg[1].blk_begin) ? 1 : 0;
  const DqSeg &sg = args.seg[si];
  const int l32 = lane & 31, h = lane >> 5;
  const int M = args.M, K = args.K, N = sg.N;
  const int nsb = K >> 8;
  const int nsteps = (nsb + C - 1) / C;
  constexpr int kPitch = C * 256 + 8;  // halves; 4 dwords mod 64 banks

  const uint32_t a_row = static_cast<uint32_t>(K >> 5) * kQ8_1Bytes;
  const uint32_t w_row = static_cast<uint32_t>(
      QT == kTypeQ8_0 ? (K >> 5) * kQ8_0Bytes : (K >> 8) * (QT == kTypeQ4_K ? kQ4KBytes : kQ6KBytes));
  const rsrc_t Wr = make_rsrc(sg.W, w_row * static_cast<uint32_t>(TL ? (N + 31) & ~31 : N));
  const rsrc_t Ar = make_rsrc(args.A, a_row * static_cast<uint32_t>(M));
  const int n = SW ? bx * 64 + (rw & 1) * 32 + l32
                   : (bx - sg.blk_begin) * kRowsPerWg + rw * 32 + l32;
  const uint32_t row_off = TL ? static_cast<uint32_t>(n >> 5) * 32 * w_row
                              : static_cast<uint32_t>(min(n, N - 1)) * w_row;
  const int stage_halves = (M + 1) * kPitch;
  const int arow_off = (l32 < M ? l32 : M) * kPitch;  // batch rows past M read the zero row M

  // the wave's super-block i (K order i * kHalves + half); past the end:
  // out of range, zeros, no reads
  auto fetch = [&](RawW<QT> &r, int i) {
    const int t = i * kHalves + half;
    fetch_w<QT, TL>(r, Wr, t < nsb ? row_off : kOobOffset, t < nsb ? t : 0, h, l32);
  };

  f32x16 acc0, acc1;
#pragma unroll
  for (int i = 0; i < 16; ++i) acc0[i] = acc1[i] = 0.0f;

  // prologue: stage 0's loads, the ring's first D - 1 super-blocks, stage 0
  StageR<C, NT> st;
  stage_r_load<C, NT>(st, Ar, a_row, M, 0, nsb, tid);
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_sched_barrier(0);
  RawW<QT> w[D];
#pragma unroll
  for (int j = 0; j < D - 1; ++j) fetch(w[j], j);
  for (int i = tid; i < kPitch / 8; i += NT) {
    reinterpret_cast<u32x4 *>(lds + M * kPitch)[i] = u32x4{0, 0, 0, 0};
    reinterpret_cast<u32x4 *>(lds + stage_halves + M * kPitch)[i] = u32x4{0, 0, 0, 0};
  }
  stage_r_store<C, NT>(st, lds, kPitch, M, tid);
  __syncthreads();
  IFX_STAMP(1);

  // one stage step; off: the ring slot of its first super-block (a constant:
  // the loop below takes D / Cw steps per pass)
  auto step = [&](auto off, int s) {
    const _Float16 *sa = lds + (s & 1) * stage_halves + arow_off;
    // the next step's activations, ahead of this step's weight loads
    stage_r_load<C, NT>(st, Ar, a_row, M, s + 1, nsb, tid);
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int u = 0; u < Cw; ++u) {
      fetch(w[(decltype(off)::value + u + D - 1) % D], s * Cw + u + D - 1);
      compute<QT>(w[(decltype(off)::value + u) % D], sa + 256 * (u * kHalves + half), h, acc0, acc1);
    }
    if (s + 1 < nsteps) stage_r_store<C, NT>(st, lds + ((s + 1) & 1) * stage_halves, kPitch, M, tid);
    __syncthreads();
    if (s < 5) IFX_STAMP(2 + s);
  };
  for (int s = 0; s < nsteps; s += D / Cw) {
    step(std::integral_constant<int, 0>{}, s);
    if constexpr (D == 2 * Cw) {
      if (s + 1 < nsteps) step(std::integral_constant<int, Cw>{}, s + 1);
    }
  }

  // lane holds column n and batch rows 8*(i/4) + 4*h + (i%4)
  float yv[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) yv[i] = acc0[i] + acc1[i];
  if constexpr (WV == 8) {
    // the second half's sums -> LDS [row slice][16][64], added by the first
    float *red = reinterpret_cast<float *>(lds) + rw * 1024 + lane;
    if (half) {
#pragma unroll
      for (int i = 0; i < 16; ++i) red[64 * i] = yv[i];
    }
    __syncthreads();
    if (!half) {
#pragma unroll
      for (int i = 0; i < 16; ++i) yv[i] += red[64 * i];
    }
  }
  if constexpr (SW) {
    // gate / up sums of the 64 outputs -> LDS [projection][batch row][64]
    // (past the stages and the halves' sums)
    float *gu = reinterpret_cast<float *>(lds) + (WV == 8 ? 4096 : 0);
    const int proj = rw >> 1, col = (rw & 1) * 32 + l32;
    if (!half) {
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int m = 8 * (i >> 2) + 4 * h + (i & 3);
        if (m < M) gu[(proj * kMaxM + m) * 64 + col] = yv[i];
      }
    }
    __syncthreads();
    const int n0 = bx * 64;
    for (int it = tid; it < M * 16; it += NT) {
      const int blk = it >> 3, l = it & 7, m = blk >> 1, b = blk & 1;
      const int o = n0 + 32 * b + 4 * l;
      if (n0 + 32 * b >= N) continue;
      const f32x4 g4 = *reinterpret_cast<const f32x4 *>(&gu[m * 64 + 32 * b + 4 * l]);
      const f32x4 u4 = *reinterpret_cast<const f32x4 *>(&gu[(kMaxM + m) * 64 + 32 * b + 4 * l]);
      const f32x4 hv = silu_mul4(g4, u4);
      const int64_t oh = static_cast<int64_t>(m) * N + o;
      if (args.H) {
        if (args.h_f16) {
          const u32x2 hh = {f2h_bits(hv.x) | (f2h_bits(hv.y) << 16),
                            f2h_bits(hv.z) | (f2h_bits(hv.w) << 16)};
          *reinterpret_cast<u32x2 *>(static_cast<uint16_t *>(args.H) + oh) = hh;
        } else {
          *reinterpret_cast<f32x4 *>(static_cast<float *>(args.H) + oh) = hv;
        }
      }
      if (args.Q)
        quantize4_store(hv.x, hv.y, hv.z, hv.w,
                        args.Q + (static_cast<int64_t>(m) * (N >> 5) + (o >> 5)) * kQ8_1Bytes, l);
    }
    IFX_STAMP(7);
    return;
  }
  IFX_STAMP(7);
  if (half || n >= N) return;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int m = 8 * (i >> 2) + 4 * h + (i & 3);
    if (m >= M) continue;
    const int64_t o = static_cast<int64_t>(m) * N + n;
    float y = yv[i];
    if constexpr (F16OUT) {
      uint16_t *Yh = static_cast<uint16_t *>(sg.Y);
      if (args.mode == 1) y += h2f(Yh[o]);
      else if (args.mode == 2) y += h2f(static_cast<const uint16_t *>(sg.bias)[n]);
      Yh[o] = static_cast<uint16_t>(f2h_bits(y));
    } else {
      float *Yf = static_cast<float *>(sg.Y);
      if (args.mode == 1) y += Yf[o];
      else if (args.mode == 2) y += static_cast<const float *>(sg.bias)[n];
      Yf[o] = y;
    }
  }
}

namespace {

// Largest K range (super-blocks) whose fp16 activation stage fits kLdsBytes.
int dq_sb_max(int M) { return max(1, (kLdsBytes / 2 / (M + 1) - 8) / 256); }

// Super-block splits: at least what the activation stage needs, and about
// 512 workgroups (two per CU on 256 CUs) up to M = 16, 320 above (fewer
// partial sums: 14B Q/K/V at M = 32 13.8 -> 13.05 us, ordered 15.6 -> 13.9,
// O 9.55 -> 9.05, ordered 13.1 -> 13.85; at M = 16 the 14B O / down lose
// 0.9 / 2.8 us with it); fp16 outputs without the ordered-split workspace
// (no_split) take the fewest the stage allows.  IFX_DQ_WGS sets the
// workgroup target (tuning; read once).
int dq_splits(int groups, int nsb, int M, bool no_split) {
  static const int env = [] {
    const char *e = ifx::tuning_env("IFX_DQ_WGS");
    return e && atoi(e) > 0 ? atoi(e) : 0;
  }();
  const int target = env ? env : M > 16 ? 320 : 512;
  const int need = (nsb + dq_sb_max(M) - 1) / dq_sb_max(M);
  if (no_split) return need;
  return max(need, min(nsb, (target + groups - 1) / groups));
}

// Launches with at least this many row groups of 128 (three quarters of
// the 256 CUs) take the no-split rolling-stage form, k_gemv_dqr: measured on
// the 14B gate/up pair (216 groups), it beats the K split with its partial
// sums.  IFX_DQR_GROUPS overrides (tuning; read once; 0 = never).
int dqr_min_groups() {
  static const int v = [] {
    const char *e = ifx::tuning_env("IFX_DQR_GROUPS");
    return e ? atoi(e) : 192;
  }();
  return v;
}

// Whether a launch of `groups` row groups takes k_gemv_dqr.
bool dq_rolling(int groups, int splits_req) {
  return dqr_min_groups() > 0 && groups >= dqr_min_groups() && splits_req == 0;
}

// Row groups and K splits of a launch (sets blk_begin and sb_per);
// rolling: the launch takes k_gemv_dqr (ks = 1, sb_per unused).
void dq_plan(DqArgs &args, bool no_split, int splits_req, int &groups, int &ks,
             bool *rolling = nullptr) {
  groups = 0;
  for (int i = 0; i < args.nseg; ++i) {
    args.seg[i].blk_begin = groups;
    groups += (args.seg[i].N + kRowsPerWg - 1) / kRowsPerWg;
  }
  const bool roll = dq_rolling(groups, splits_req);
  if (rolling) *rolling = roll;
  if (roll) {
    ks = 1;
    args.sb_per = args.K >> 8;
    return;
  }
  const int nsb = args.K >> 8;
  const int need = (nsb + dq_sb_max(args.M) - 1) / dq_sb_max(args.M);
  ks = (splits_req > 0 && !no_split) ? max(need, min(splits_req, nsb))
                                     : dq_splits(groups, nsb, args.M, no_split);
  args.sb_per = (nsb + ks - 1) / ks;
  ks = (nsb + args.sb_per - 1) / args.sb_per;
}


// The no-split rolling-stage launch (k_gemv_dqr): C super-blocks per stage
// step (M * 8 * C <= 1024 Q8_1 blocks, two stages within 160 KB), D in
// flight per wave.  groups: row groups of 128 (SW: pairs of 64 outputs).
template <int QT, bool F16, bool TL, bool SW, int C, int D, int WV>
hipError_t launch_dqr_c(const DqArgs &args, int groups, hipStream_t s) {
  constexpr int kPitch = C * 256 + 8;
  constexpr int kMaxMr = 1024 / (8 * C);  // the stage's batch rows
  if (args.M > kMaxMr) return hipErrorInvalidValue;
  const size_t shm = std::max(static_cast<size_t>(2) * (args.M + 1) * kPitch * 2,
                              static_cast<size_t>(2 * 4096 * 4));  // halves' sums + gate/up sums
  if (!dry_run()) {
    static const hipError_t attr = hipFuncSetAttribute(
        reinterpret_cast<const void *>(&k_gemv_dqr<QT, F16, TL, SW, C, D, WV>),
        hipFuncAttributeMaxDynamicSharedMemorySize,
        static_cast<int>(std::max(2 * (kMaxMr + 1) * kPitch * 2, 2 * 4096 * 4)));
    if (attr != hipSuccess) return attr;
  }
  IFX_LAUNCH(k_gemv_dqr, (QT, F16, TL, SW, C, D, WV), dim3(groups), dim3(64 * WV), shm, s, args);
  return last_error();
}

// 8 waves (two per row slice: 26.9 against 28.2 us for one, fused 14B
// gate/up at M = 32); C = 4 super-blocks a stage step above M = 16, 8 up to
// it; D = C / 2 super-blocks in flight per wave (D = C measured the same,
// with a longer prologue).  Q8_0 (40 registers a super-block) keeps C = 4
// and D = 2 at every M: with 8 and 4 it runs one wave per SIMD (LM head
// 151936 x 2048 at M = 16: 90.8 us, against 75.3 on this form and 82.9 on
// the K split).
template <int QT, bool F16, bool TL, bool SW>
hipError_t launch_dqr(const DqArgs &args, int groups, hipStream_t s) {
  if (args.M > 16 || QT == kTypeQ8_0) return launch_dqr_c<QT, F16, TL, SW, 4, 2, 8>(args, groups, s);
  return launch_dqr_c<QT, F16, TL, SW, 8, 4, 8>(args, groups, s);
}


template <int QT, bool TL>
hipError_t launch_qt(DqArgs args, bool f16, int splits_req, hipStream_t s) {
  const bool ordered = args.ws.cnt != nullptr;
  int groups = 0, ks = 1;
  bool rolling = false;
  dq_plan(args, f16 && !ordered, splits_req, groups, ks, &rolling);
  if (rolling) {
    if (f16) return launch_dqr<QT, true, TL, false>(args, groups, s);
    return launch_dqr<QT, false, TL, false>(args, groups, s);
  }
  // fp16 sums cannot be added with atomics: split only through the workspace
  if (f16 && ks > 1 && !ordered) return hipErrorInvalidValue;
  const size_t shm = static_cast<size_t>(args.M + 1) * (args.sb_per * 256 + 8) * 2;
  const dim3 grid(groups, ks), block(64 * kWaves);
  if (f16 && ks > 1) {
    if constexpr (TL) IFX_LAUNCH(k_gemv_dq, (QT, true, 2, true), grid, block, shm, s, args);
    else IFX_LAUNCH(k_gemv_dq, (QT, true, 2), grid, block, shm, s, args);
  } else if (f16) {
    if constexpr (TL) IFX_LAUNCH(k_gemv_dq, (QT, true, 0, true), grid, block, shm, s, args);
    else IFX_LAUNCH(k_gemv_dq, (QT, true, 0), grid, block, shm, s, args);
  } else if (ks == 1) {
    if constexpr (TL) IFX_LAUNCH(k_gemv_dq, (QT, false, 0, true), grid, block, shm, s, args);
    else IFX_LAUNCH(k_gemv_dq, (QT, false, 0), grid, block, shm, s, args);
  } else if (ordered) {
    if constexpr (TL) IFX_LAUNCH(k_gemv_dq, (QT, false, 2, true), grid, block, shm, s, args);
    else IFX_LAUNCH(k_gemv_dq, (QT, false, 2), grid, block, shm, s, args);
  } else {
    if (args.mode != 1) {  // store / bias: the splits add into zeroed outputs
      FillArgs f{};
      for (int i = 0; i < args.nseg; ++i) {
        f.y[i] = static_cast<float *>(args.seg[i].Y);
        f.n[i] = static_cast<int64_t>(args.M) * args.seg[i].N;
      }
      if (launch_fill_zero(f, args.nseg, s) != hipSuccess) return last_error();
    }
    if constexpr (TL) IFX_LAUNCH(k_gemv_dq, (QT, false, 1, true), grid, block, shm, s, args);
    else IFX_LAUNCH(k_gemv_dq, (QT, false, 1), grid, block, shm, s, args);
  }
  return last_error();
}

}  // namespace

namespace {

template <int QT, bool TL>
hipError_t launch_sw(const DqArgs &args, int groups, int ks, hipStream_t s) {
  const size_t stage = static_cast<size_t>(args.M + 1) * (args.sb_per * 256 + 8) * 2;
  const size_t shm = std::max(stage, static_cast<size_t>(2 * kMaxM * 64 * 4));  // + gate/up sums
  const dim3 grid(groups, ks), block(64 * kWaves);
  if (ks == 1) IFX_LAUNCH(k_gemv_dq, (QT, false, 0, TL, true), grid, block, shm, s, args);
  else IFX_LAUNCH(k_gemv_dq, (QT, false, 2, TL, true), grid, block, shm, s, args);
  return last_error();
}

// The pair plan (gate and up as one grouped launch of two projections):
// row groups, K splits and sb_per as the grouped launch chooses them.
void sw_plan(DqArgs &args, int N, int &pair_groups, int &ks, bool *rolling = nullptr) {
  args.seg[0].N = args.seg[1].N = N;
  args.nseg = 2;
  dq_plan(args, false, 0, pair_groups, ks, rolling);
}

}  // namespace

bool gemv_dq_fits(int qtype, int M, int K);

// K splits of the fused gate/up/SiLU launch (1: no workspace needed).
int gemv_dq_swiglu_splits(int M, int N, int K) {
  DqArgs args{};
  args.M = M;
  args.K = K;
  int pg = 0, ks = 1;
  sw_plan(args, N, pg, ks);
  return ks;
}

// Fused gate/up/SiLU on the fp16-dequant GEMV (k_gemv_dq, SW); N % 32 == 0.
// ws: the pair's ordered-split workspace (gemv_dq_workspace_bytes of
// count 2, N, N), required when the launch splits K.
hipError_t launch_gemv_dq_swiglu(int qtype, const void *Wg, const void *Wu, const void *A,
                                 void *H, bool h_f16, void *Q, int M, int N, int K, void *ws,
                                 hipStream_t stream) {
  if (!gemv_dq_fits(qtype, M, K) || N % 32 != 0) return hipErrorInvalidValue;
  DqArgs args{};
  args.seg[0] = DqSeg{static_cast<const uint8_t *>(Wg), nullptr, nullptr, N, 0};
  args.seg[1] = DqSeg{static_cast<const uint8_t *>(Wu), nullptr, nullptr, N, 0};
  args.A = static_cast<const uint8_t *>(A);
  args.M = M;
  args.K = K;
  args.mode = 0;
  args.H = H;
  args.Q = static_cast<uint8_t *>(Q);
  args.h_f16 = h_f16 ? 1 : 0;
  int pair_groups = 0, ks = 1;
  bool rolling = false;
  sw_plan(args, N, pair_groups, ks, &rolling);
  const int groups = (N + 63) / 64;
  if (rolling) {
    switch (qtype) {
    case kTypeQ4_K: return launch_dqr<kTypeQ4_K, false, false, true>(args, groups, stream);
    case kTypeQ6_K: return launch_dqr<kTypeQ6_K, false, false, true>(args, groups, stream);
    case kTypeQ8_0: return launch_dqr<kTypeQ8_0, false, false, true>(args, groups, stream);
    case kTypeQ4_KT: return launch_dqr<kTypeQ4_K, false, true, true>(args, groups, stream);
    case kTypeQ6_KT: return launch_dqr<kTypeQ6_K, false, true, true>(args, groups, stream);
    case kTypeQ8_0T: return launch_dqr<kTypeQ8_0, false, true, true>(args, groups, stream);
    default: return hipErrorInvalidValue;
    }
  }
  if (ks > 1) {
    if (!ws) return hipErrorInvalidValue;
    // the pair's workspace layout: counters for its row groups, then slots
    args.ws.cnt = static_cast<uint32_t *>(ws);
    args.ws.part = reinterpret_cast<float *>(static_cast<uint8_t *>(ws) +
                                             (static_cast<int64_t>(pair_groups) * 4 + 255) / 256 * 256);
  }
  switch (qtype) {
  case kTypeQ4_K: return launch_sw<kTypeQ4_K, false>(args, groups, ks, stream);
  case kTypeQ6_K: return launch_sw<kTypeQ6_K, false>(args, groups, ks, stream);
  case kTypeQ8_0: return launch_sw<kTypeQ8_0, false>(args, groups, ks, stream);
  case kTypeQ4_KT: return launch_sw<kTypeQ4_K, true>(args, groups, ks, stream);
  case kTypeQ6_KT: return launch_sw<kTypeQ6_K, true>(args, groups, ks, stream);
  case kTypeQ8_0T: return launch_sw<kTypeQ8_0, true>(args, groups, ks, stream);
  default: return hipErrorInvalidValue;
  }
}

// Types and batch sizes of the fp16-dequant GEMV.
bool gemv_dq_fits(int qtype, int M, int K) {
  return (qtype == kTypeQ4_K || qtype == kTypeQ6_K || qtype == kTypeQ8_0 || qtype == kTypeQ4_KT ||
          qtype == kTypeQ6_KT || qtype == kTypeQ8_0T) && M >= 1 &&
         M <= kMaxM && K % 256 == 0;
}

// fp16 outputs of the split form without a workspace: one activation stage
// holds K.
bool gemv_dq_fits_f16(int M, int K) { return M <= kMaxM && K / 256 <= dq_sb_max(M); }
// ... or the launch (count projections of N rows) takes the no-split form.
bool gemv_dq_f16_unsplit(int count, const int *N, int M, int K) {
  int groups = 0;
  for (int i = 0; i < count; ++i) groups += (N[i] + kRowsPerWg - 1) / kRowsPerWg;
  return M <= kMaxM && (K / 256 <= dq_sb_max(M) || dq_rolling(groups, 0));
}

// count projections (1..3) of one quant type share A; bias only with
// count == 1.  splits_req: 0 = chosen from the shape.
// Workspace bytes of the ordered split (0: the launch does not split):
// counters (256-byte aligned) then one 16 KB slot per (row group, split).
int64_t gemv_dq_workspace_bytes(int count, const int *N, bool f16, int M, int K) {
  DqArgs args{};
  for (int i = 0; i < count; ++i) args.seg[i].N = N[i];
  args.nseg = count;
  args.M = M;
  args.K = K;
  int groups = 0, ks = 1;
  (void)f16;  // fp16 outputs split as fp32 ones when the workspace is given
  dq_plan(args, false, 0, groups, ks);
  if (ks <= 1) return 0;
  return (static_cast<int64_t>(groups) * 4 + 255) / 256 * 256 +
         static_cast<int64_t>(groups) * ks * kWaves * 64 * 16 * 4;
}

// ws: the ordered-split workspace (gemv_dq_workspace_bytes, counters zero),
// or nullptr for atomics.
hipError_t launch_gemv_dq(int qtype, int count, const void *const *W, void *const *Y,
                          const int *N, const void *bias, const void *A, bool f16, int M, int K,
                          int mode, int splits_req, hipStream_t stream, void *ws) {
  if (!gemv_dq_fits(qtype, M, K) || count < 1 || count > 3) return hipErrorInvalidValue;
  DqArgs args{};
  if (ws) {
    int groups = 0;
    for (int i = 0; i < count; ++i) groups += (N[i] + kRowsPerWg - 1) / kRowsPerWg;
    args.ws.cnt = static_cast<uint32_t *>(ws);
    args.ws.part = reinterpret_cast<float *>(static_cast<uint8_t *>(ws) +
                                             (static_cast<int64_t>(groups) * 4 + 255) / 256 * 256);
  }
  for (int i = 0; i < count; ++i)
    args.seg[i] = DqSeg{static_cast<const uint8_t *>(W[i]), Y[i], i == 0 ? bias : nullptr, N[i], 0};
  args.nseg = count;
  args.A = static_cast<const uint8_t *>(A);
  args.M = M;
  args.K = K;
  args.mode = mode;
  switch (qtype) {
  case kTypeQ4_K: return launch_qt<kTypeQ4_K, false>(args, f16, splits_req, stream);
  case kTypeQ6_K: return launch_qt<kTypeQ6_K, false>(args, f16, splits_req, stream);
  case kTypeQ8_0: return launch_qt<kTypeQ8_0, false>(args, f16, splits_req, stream);
  case kTypeQ4_KT: return launch_qt<kTypeQ4_K, true>(args, f16, splits_req, stream);
  case kTypeQ6_KT: return launch_qt<kTypeQ6_K, true>(args, f16, splits_req, stream);
  case kTypeQ8_0T: return launch_qt<kTypeQ8_0, true>(args, f16, splits_req, stream);
  default: return hipErrorInvalidValue;
  }
}

}  // namespace ifx

#ifdef IFX_STAMPS
// Tuning builds: the wave timeline records of this file's kernels (8 int64
// per wave, see IFX_STAMP) copied to host memory, then cleared; returns the
// record count.
extern "C" int ifx_debug_stamps_dq(long long *out, int max_waves) {
  const int n = max_waves < ifx::kStampWaves ? max_waves : ifx::kStampWaves;
  void *p = nullptr;
  if (hipGetSymbolAddress(&p, HIP_SYMBOL(ifx::ifx_stamps)) != hipSuccess) return -1;
  if (hipMemcpy(out, p, static_cast<size_t>(n) * 64, hipMemcpyDeviceToHost) != hipSuccess) return -1;
  if (hipMemset(p, 0, static_cast<size_t>(ifx::kStampWaves) * 64) != hipSuccess) return -1;
  return n;
}
#endif
