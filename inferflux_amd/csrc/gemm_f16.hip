// gemm_f16.hip -- prefill GEMM on the fp16 matrix cores of gfx950, with the
// weights dequantized inside the kernel: y[m][n] = sum_k W[n][k] * x[m][k],
// W raw GGUF Q4_K / Q6_K / Q8_0 blocks, x given as Q8_1 blocks of 32,
// fp32 accumulate.
//
// This is the arithmetic of the reference's prefill path, fused: above its
// MMQ limit the reference dequantizes W to an FP16 scratch copy
// (runtime/backends/cuda/native/quantized_weight_map.cpp:176-233, element
// formulas kernels/quant_common.cuh:100-188) and multiplies it with cuBLAS
// in FP16 with fp32 accumulation (cublas_gemm.h:47, called at
// transformer_forward.cu:1479).  Here the FP16 copy never exists: each
// workgroup dequantizes the 64-value K slice of its 256 weight rows into
// LDS, next to the matching 256 activation rows (Q8_1 codes times their
// block scale, rounded to fp16), and v_mfma_f32_32x32x16_f16 multiplies
// them.  Per element, w = fp16(d*sc) * q - fp16(dmin*m) (Q4_K),
// fp16(d*sc) * (q - 32) (Q6_K), fp16(d) * q (Q8_0), each one fp16 fused
// multiply-add or multiply; x = fp16(d_a) * q_a.  The rounding of w and x to
// fp16 (relative 2^-11) is the reference's own FP16 prefill rounding; the
// integer-exact int8 kernel (gemm_mfma.hip) remains for mid-size batches.
//
// Why not int8: the per-32-value rescale of int8 MFMA results costs three
// VALU operations per output per block and bounds that kernel near 15 % of
// the int8 peak.  Dequantizing to fp16 costs about two VALU operations per
// weight element per workgroup pass instead, independent of M.
//
// Workgroup: 512 threads (8 waves, 4 along m x 2 along n), output tile 256
// (m) x 256 (n); each wave owns 64 x 128 = 2 x 4 MFMA tiles of 32 x 32
// (128 fp32 accumulators per lane).  The K loop steps 64 values:
//   * LDS holds two stages (double buffer, 2 x 72 KB): while the waves run
//     the 32 MFMAs of stage c from one buffer, they convert the raw bytes of
//     stage c+1 (already in registers) into the other buffer and issue the
//     global loads of stage c+2; one barrier per step.
//   * Packed fp16 dequant: four code bytes become two fp16 pairs with one
//     and-or each, (0x6400 | b) = 1024 + b, then v_pk_add / v_pk_fma.  The
//     pairs hold values (0, 2) and (1, 3) of each group of four; both
//     operands are stored in that order, so the K permutation cancels in
//     the dot product.
// Launch: the workgroup index is remapped so that workgroups on one XCD
// (hardware round-robin over 8 XCDs) take consecutive tiles, sharing weight
// tiles in that XCD's L2.  When the tile grid alone cannot fill the chip
// (e.g. N = 5120, M = 512: 40 tiles), K is split over workgroups whose fp32
// partial sums are added into Y with atomics (after a zero fill in store
// mode), as the split-K decode kernels do.
// MFMA lane layouts (32x32x16 f16): lane l supplies row (l % 32) of A and
// column (l % 32) of B, with 8 K values for K half l / 32; it receives
// column l % 32 and rows 8*(i/4) + 4*(l/32) + (i%4), i = 0..15.
#include "../../include/ifx_qgemm.h"
#include "ifx_common.h"

#include <mutex>

namespace ifx {

namespace {

typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef _Float16 h8 __attribute__((ext_vector_type(8)));

constexpr int kBM = 256, kBN = 256, kBK = 64;
// A staged row is its 64 K values as eight 16-byte groups, unpadded; group
// g of row r sits at position g ^ swz(r).  The swizzle makes both access
// patterns conflict-free on 64 banks (16 lanes per b128 phase) and on 32
// banks (8 lanes): the MFMA operand reads (lane l: row l % 32, group
// 2 ks + l / 32) and the stage writes (threads 2r, 2r + 1: both halves of
// row r, activations groups 4 p + j, Q4_K / Q6_K weights 2 p, 2 p + 1,
// 4 + 2 p, 5 + 2 p).  With a 72-half padded pitch and no swizzle the writes
// were 2-way conflicted (counters: about one conflict cycle per LDS
// instruction).  The table was found by exhaustive search over the two bank
// models.
constexpr int kPitch = kBK;  // halves per staged row
__device__ __forceinline__ int swz(int r) {
  // (r & 1) ^ g[(r >> 1) & 7] with g = {0, 6, 3, 5, 1, 7, 2, 4}
  return (r & 1) ^ ((0x8B9AF0 >> (3 * ((r >> 1) & 7))) & 7);
}
// Halves offset of group g of row r in a stage buffer.
__device__ __forceinline__ int slot(int r, int g) { return r * kPitch + 8 * (g ^ swz(r)); }
#ifndef IFX_F16_VALU_PER_MFMA
#define IFX_F16_VALU_PER_MFMA 5
#endif
#ifndef IFX_F16_WAVES
#define IFX_F16_WAVES 8
#endif

struct Smem {
  _Float16 a[2][kBM * kPitch];  // activations [m][k slot]
  _Float16 w[2][kBN * kPitch];  // weights [n][k slot]
};

constexpr uint32_t kMagic = 0x64006400u;  // fp16 1024.0 in both halves

__device__ __forceinline__ h2 as_h2(uint32_t u) { return __builtin_bit_cast(h2, u); }
__device__ __forceinline__ uint32_t as_u32(h2 h) { return __builtin_bit_cast(uint32_t, h); }
__device__ __forceinline__ h2 splat(float f) {
  const _Float16 h = static_cast<_Float16>(f);
  return h2{h, h};
}

// Raw bytes of one 64-value stage for one thread: activation block
// (row tid/2, block tid&1 of the stage) and a weight half-row or block.
template <int QT>
struct Raw {
  uint32_t ads;     // Q8_1 {d, s}
  u32x4 a0, a1;     // Q8_1 codes; fp16 activations (AH): the block's 64 bytes in a0..a3
  u32x4 a2, a3;
  u32x4 w0, w1;     // Q4_K: header, 16 qs bytes; Q6_K: ql, qh; Q8_0: codes 0-15, 16-31
  uint32_t wx0, wx1;  // Q4_K: stage c & 3; Q6_K: 4 scale bytes, d; Q8_0: -, d
};

// Q8_1 blocks of stage c (64 values): first and second 32-value half.
// Q4_K: sub-blocks 2p, 2p+1 of super-block c/4 (they share qs bytes).
// Q6_K: sub-blocks hf and hf + 2 of 128-value half g (they share ql/qh
// bytes), c = 4*sb + 2*g + hf.  Q8_0: blocks 2c, 2c+1.
template <int QT>
__device__ __forceinline__ int stage_block(int c, int half) {
  if constexpr (QT == kTypeQ6_K) {
    const int sb = c >> 2, g = (c >> 1) & 1, hf = c & 1;
    return sb * 8 + g * 4 + hf + 2 * half;
  } else {
    return 2 * c + half;
  }
}

template <int QT, bool AH>
__device__ __forceinline__ void fetch(Raw<QT> &r, rsrc_t Wr, rsrc_t Ar, uint32_t w_off,
                                      uint32_t a_off, int c, int part) {
  // activation block: row (tid >> 1), half `part`
  if constexpr (AH) {  // already converted: 32 fp16 values in commit's order
    const uint32_t o = a_off + stage_block<QT>(c, part) * 64;
    r.a0 = bload<u32x4>(Ar, o, 0);
    r.a1 = bload<u32x4>(Ar, o + 16, 0);
    r.a2 = bload<u32x4>(Ar, o + 32, 0);
    r.a3 = bload<u32x4>(Ar, o + 48, 0);
  } else {
    const uint32_t o = a_off + stage_block<QT>(c, part) * kQ8_1Bytes;
    r.ads = bload<uint32_t>(Ar, o, 0);
    r.a0 = bload<u32x4>(Ar, o + 4, 0);
    r.a1 = bload<u32x4>(Ar, o + 20, 0);
  }
  if constexpr (QT == kTypeQ4_K) {
    const uint32_t o = w_off + (c >> 2) * kQ4KBytes;
    r.w0 = wload<u32x4>(Wr, o, 0);
    r.w1 = wload<u32x4>(Wr, o + 16 + (c & 3) * 32 + 16 * part, 0);
  } else if constexpr (QT == kTypeQ6_K) {
    const int g = (c >> 1) & 1, hf = c & 1;
    const uint32_t o = w_off + (c >> 2) * kQ6KBytes;
    r.w0 = wload<u32x4>(Wr, o + g * 64 + hf * 32 + 16 * part, 0);
    r.w1 = wload<u32x4>(Wr, o + 128 + g * 32 + 16 * part, 0);
    const u32x2 sc = wload<u32x2>(Wr, o + 192 + g * 8, 0);
    r.wx0 = (hf ? (sc.x >> 16) | (sc.y & 0xFFFF0000u) : (sc.x & 0xFFFFu) | (sc.y << 16));
    // r.wx0 bytes: [sc(hf), part 0], [part 1], [sc(hf+2), part 0], [part 1]
    r.wx1 = wload<uint16_t>(Wr, o + 208, 0);
  } else {
    const uint32_t o = w_off + (2 * c + part) * kQ8_0Bytes;
    r.wx1 = wload<uint16_t>(Wr, o, 0);
    r.w0 = wload<u32x4>(Wr, o + 2, 0);
    r.w1 = wload<u32x4>(Wr, o + 18, 0);
  }
}

// Signed byte codes (four per word) times scale d -> two fp16 pairs holding
// values (0, 2) and (1, 3).  q ^ 0x80 = q + 128 as an unsigned byte, so
// (0x6400 | byte) - 1152 = q exactly; the product is rounded once.
__device__ __forceinline__ void i8x4_to_h(uint32_t x, h2 d, uint32_t &p02, uint32_t &p13) {
  const uint32_t mg = vreg(kMagic);
  x ^= 0x80808080u;
  const h2 off = {static_cast<_Float16>(-1152.0f), static_cast<_Float16>(-1152.0f)};
  const h2 a = as_h2((x & 0x00FF00FFu) | mg) + off;
  const h2 b = as_h2(((x >> 8) & 0x00FF00FFu) | mg) + off;
  p02 = as_u32(a * d);
  p13 = as_u32(b * d);
}

// Unsigned byte codes v (< 1024) -> fp16 pairs of (v + bias) * d - mn.
__device__ __forceinline__ void u8x4_to_h(uint32_t x, h2 bias, h2 d, h2 mn, uint32_t &p02,
                                          uint32_t &p13) {
  const uint32_t mg = vreg(kMagic);
  const h2 a = as_h2((x & 0x00FF00FFu) | mg) + bias;
  const h2 b = as_h2(((x >> 8) & 0x00FF00FFu) | mg) + bias;
  p02 = as_u32(__builtin_elementwise_fma(a, d, -mn));
  p13 = as_u32(__builtin_elementwise_fma(b, d, -mn));
}

// Nibble codes of a word of packed 4-bit codes (HI = 0: low, 1: high
// nibbles) -> fp16 pairs q * d - mn of bytes (0, 2) and (1, 3).  Low
// nibbles sit in mantissa bits 0..3 under the magic 1024 (ulp 1): 1024 + q;
// high nibbles stay in bits 4..7, under the magic 64 (0x5400, ulp 1/16)
// also exactly 64 + q, so neither needs more than the one shift by 8.
template <int HI>
__device__ __forceinline__ void q4x4_to_h(uint32_t x, h2 d, h2 mn, uint32_t &p02, uint32_t &p13) {
  constexpr uint32_t msk = HI ? 0x00F000F0u : 0x000F000Fu;
  const uint32_t mg = vreg(HI ? 0x54005400u : kMagic);
  const h2 bias = splat(HI ? -64.0f : -1024.0f);
  const h2 a = as_h2((x & msk) | mg) + bias;
  const h2 b = as_h2(((x >> 8) & msk) | mg) + bias;
  p02 = as_u32(__builtin_elementwise_fma(a, d, -mn));
  p13 = as_u32(__builtin_elementwise_fma(b, d, -mn));
}

// The 32 activation values of one Q8_1 block as fp16, in the order the GEMM
// stores them: word 2j / 2j+1 holds values (4j, 4j+2) / (4j+1, 4j+3).
__device__ __forceinline__ void q8_1_block_to_h(uint32_t ads, u32x4 a0, u32x4 a1, uint32_t (&o)[16]) {
  const h2 d = splat(h2f(ads & 0xFFFFu));
  const uint32_t in[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
#pragma unroll
  for (int j = 0; j < 8; ++j) i8x4_to_h(in[j], d, o[2 * j], o[2 * j + 1]);
}

// Convert one stage's raw bytes and store them in LDS buffer `buf`.
template <int QT, bool AH>
__device__ __forceinline__ void commit(Smem &sm, int buf, const Raw<QT> &r, int item) {
  const int row = item >> 1, part = item & 1;
  if constexpr (AH) {
    _Float16 *arow = sm.a[buf];
    *reinterpret_cast<u32x4 *>(arow + slot(row, 4 * part)) = r.a0;
    *reinterpret_cast<u32x4 *>(arow + slot(row, 4 * part + 1)) = r.a1;
    *reinterpret_cast<u32x4 *>(arow + slot(row, 4 * part + 2)) = r.a2;
    *reinterpret_cast<u32x4 *>(arow + slot(row, 4 * part + 3)) = r.a3;
  } else {  // activations: 32 values of block `part` at slots 32*part ..
    uint32_t o[16];
    q8_1_block_to_h(r.ads, r.a0, r.a1, o);
    _Float16 *arow = sm.a[buf];
#pragma unroll
    for (int j = 0; j < 4; ++j)
      *reinterpret_cast<u32x4 *>(arow + slot(row, 4 * part + j)) =
          u32x4{o[4 * j], o[4 * j + 1], o[4 * j + 2], o[4 * j + 3]};
  }
  _Float16 *wbuf = sm.w[buf];
  if constexpr (QT == kTypeQ4_K) {
    // 16 qs bytes: values 16*part .. +15 of sub-blocks 2p (low nibbles) and
    // 2p + 1 (high nibbles); get_scale_min_k4 (quant_common.cuh:83-94).
    const float d = h2f(r.w0.x & 0xFFFFu), dmin = h2f(r.w0.x >> 16);
    const int p = static_cast<int>(r.wx0);  // stage index within the super-block
    const uint32_t S0 = r.w0.y, S1 = r.w0.z, S2 = r.w0.w;
    const uint32_t sc_lo = S0 & 0x3F3F3F3Fu, m_lo = S1 & 0x3F3F3F3Fu;
    const uint32_t sc_hi = (S2 & 0x0F0F0F0Fu) | ((S0 >> 2) & 0x30303030u);
    const uint32_t m_hi = ((S2 >> 4) & 0x0F0F0F0Fu) | ((S1 >> 2) & 0x30303030u);
    // sub-blocks j = 2p, 2p+1: bytes (2p)&3, (2p+1)&3 of the lo (p < 2) or hi word
    const uint32_t scw = p < 2 ? sc_lo : sc_hi, mw = p < 2 ? m_lo : m_hi;
    const int sh = 16 * (p & 1);
    const float sc0 = static_cast<float>((scw >> sh) & 0xFFu);
    const float sc1 = static_cast<float>((scw >> (sh + 8)) & 0xFFu);
    const float m0 = static_cast<float>((mw >> sh) & 0xFFu);
    const float m1 = static_cast<float>((mw >> (sh + 8)) & 0xFFu);
    const h2 d0 = splat(d * sc0), d1 = splat(d * sc1);
    const h2 n0 = splat(dmin * m0), n1 = splat(dmin * m1);
    uint32_t lo[8], hi[8];
    const uint32_t in[4] = {r.w1.x, r.w1.y, r.w1.z, r.w1.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      q4x4_to_h<0>(in[j], d0, n0, lo[2 * j], lo[2 * j + 1]);
      q4x4_to_h<1>(in[j], d1, n1, hi[2 * j], hi[2 * j + 1]);
    }
    *reinterpret_cast<u32x4 *>(wbuf + slot(row, 2 * part)) = u32x4{lo[0], lo[1], lo[2], lo[3]};
    *reinterpret_cast<u32x4 *>(wbuf + slot(row, 2 * part + 1)) = u32x4{lo[4], lo[5], lo[6], lo[7]};
    *reinterpret_cast<u32x4 *>(wbuf + slot(row, 4 + 2 * part)) = u32x4{hi[0], hi[1], hi[2], hi[3]};
    *reinterpret_cast<u32x4 *>(wbuf + slot(row, 5 + 2 * part)) = u32x4{hi[4], hi[5], hi[6], hi[7]};
  } else if constexpr (QT == kTypeQ6_K) {
    // ql (w0) and qh (w1) bytes of values 16*part .. +15 of sub-blocks hf
    // (low nibbles, qh bits 2hf..2hf+1) and hf + 2 (high nibbles, qh bits
    // 2hf+4..2hf+5); dequant_q6k_element (quant_common.cuh:161-177).
    const float d = h2f(r.wx1);
    const uint32_t scb = r.wx0;
    const float s_lo = static_cast<float>(static_cast<int8_t>((scb >> (8 * part)) & 0xFFu));
    const float s_hi = static_cast<float>(static_cast<int8_t>((scb >> (16 + 8 * part)) & 0xFFu));
    const h2 dl = splat(d * s_lo), dh = splat(d * s_hi);
    const h2 b = splat(-1056.0f), zero = splat(0.0f);
    const uint32_t ql[4] = {r.w0.x, r.w0.y, r.w0.z, r.w0.w};
    const uint32_t qh[4] = {r.w1.x, r.w1.y, r.w1.z, r.w1.w};
    uint32_t lo[8], hi[8];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t y = qh[j];  // shifted right by 2*hf when fetched
      const uint32_t clo = (ql[j] & 0x0F0F0F0Fu) | ((y << 4) & 0x30303030u);
      const uint32_t chi = ((ql[j] >> 4) & 0x0F0F0F0Fu) | (y & 0x30303030u);
      u8x4_to_h(clo, b, dl, zero, lo[2 * j], lo[2 * j + 1]);
      u8x4_to_h(chi, b, dh, zero, hi[2 * j], hi[2 * j + 1]);
    }
    *reinterpret_cast<u32x4 *>(wbuf + slot(row, 2 * part)) = u32x4{lo[0], lo[1], lo[2], lo[3]};
    *reinterpret_cast<u32x4 *>(wbuf + slot(row, 2 * part + 1)) = u32x4{lo[4], lo[5], lo[6], lo[7]};
    *reinterpret_cast<u32x4 *>(wbuf + slot(row, 4 + 2 * part)) = u32x4{hi[0], hi[1], hi[2], hi[3]};
    *reinterpret_cast<u32x4 *>(wbuf + slot(row, 5 + 2 * part)) = u32x4{hi[4], hi[5], hi[6], hi[7]};
  } else {
    // one Q8_0 block (32 values) at slots 32*part ..; dequant_q8_0_element
    // (quant_common.cuh:185-188)
    const h2 d = splat(h2f(r.wx1));
    uint32_t o[16];
    const uint32_t in[8] = {r.w0.x, r.w0.y, r.w0.z, r.w0.w, r.w1.x, r.w1.y, r.w1.z, r.w1.w};
#pragma unroll
    for (int j = 0; j < 8; ++j) i8x4_to_h(in[j], d, o[2 * j], o[2 * j + 1]);
#pragma unroll
    for (int j = 0; j < 4; ++j)
      *reinterpret_cast<u32x4 *>(wbuf + slot(row, 4 * part + j)) =
          u32x4{o[4 * j], o[4 * j + 1], o[4 * j + 2], o[4 * j + 3]};
  }
}

}  // namespace

// grid.x = n_tiles * splits * m_tiles (remapped per XCD), block 64 * WV.
// WV = 8: waves 4 (m) x 2 (n), each 64 x 128 (2 x 4 MFMA tiles);
// WV = 4: waves 2 x 2, each 128 x 128 (4 x 4 tiles, accumulators in AGPRs),
// a third less LDS operand traffic per MFMA and twice the conversion work
// per thread.
// Each workgroup covers K stages [split * cps, min(nst, (split + 1) * cps)).
// SPL: 0 one split; 1 K splits added into Y with fp32 atomics; 2 K splits
// stored to their own slots (Y = the slots, split s at Y + s * M * N, no
// epilogue; k_split_sum adds them in split order).
template <int QT, int WV, bool F16OUT, int SPL, bool AH>
__global__ __launch_bounds__(64 * WV, 1) void k_gemm_f16(const uint8_t *__restrict__ W,
                                                         const uint8_t *__restrict__ A,
                                                         void *__restrict__ Y,
                                                         const void *__restrict__ bias, int M,
                                                         int N, int K, int mode, int m_tiles,
                                                         int splits, int cps) {
  constexpr int kT = 64 * WV;            // threads
  constexpr int kFM = WV == 8 ? 2 : 4;   // MFMA tiles per wave along m
  constexpr int kWM = 32 * kFM;          // wave rows along m
  constexpr int kIpt = 2 * kBN / kT;     // (row, half) items per thread
  extern __shared__ __attribute__((aligned(16))) uint8_t smem_raw[];
  Smem &sm = *reinterpret_cast<Smem *>(smem_raw);
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int wm = WV == 8 ? (wave & 3) : (wave & 1), wn = WV == 8 ? (wave >> 2) : (wave >> 1);
  const int l32 = lane & 31, h = lane >> 5;

  // XCD-aware tile order: workgroup b runs on XCD b % 8; give each XCD a
  // contiguous run of the (n, split, m) tile sequence.
  const int total = gridDim.x;
  int b = blockIdx.x;
  if ((total & 7) == 0) b = (b & 7) * (total >> 3) + (b >> 3);
  const int mt = b % m_tiles;
  const int rest = b / m_tiles;
  const int split = rest % splits, nt = rest / splits;
  const int m0 = mt * kBM, n0 = nt * kBN;
  const int nst = K / kBK;
  const int c_begin = split * cps;
  const int c_end = min(nst, c_begin + cps);

  const int nblk32 = K >> 5;
  // AH: A holds fp16 activations (64 bytes per 32-value block)
  const uint32_t a_row = static_cast<uint32_t>(nblk32) * (AH ? 64 : kQ8_1Bytes);
  const uint32_t w_row =
      static_cast<uint32_t>(QT == kTypeQ8_0 ? nblk32 * kQ8_0Bytes
                                            : (K >> 8) * (QT == kTypeQ4_K ? kQ4KBytes : kQ6KBytes));
  const rsrc_t Wr = make_rsrc(W, w_row * static_cast<uint32_t>(N));
  const rsrc_t Ar = make_rsrc(A, a_row * static_cast<uint32_t>(M));
  const int part = tid & 1;
  // Rows past M or N repeat the last row: their outputs are never stored.
  uint32_t a_off[kIpt], w_off[kIpt];
#pragma unroll
  for (int u = 0; u < kIpt; ++u) {
    const int row = (tid >> 1) + (kT / 2) * u;
    a_off[u] = min(m0 + row, M - 1) * a_row;
    w_off[u] = min(n0 + row, N - 1) * w_row;
  }

  f32x16 acc[kFM][4];
#pragma unroll
  for (int i = 0; i < kFM; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;

  auto fetch_stage = [&](Raw<QT> *r, int c) {
#pragma unroll
    for (int u = 0; u < kIpt; ++u) {
      fetch<QT, AH>(r[u], Wr, Ar, w_off[u], a_off[u], c, part);
      if constexpr (QT == kTypeQ4_K) r[u].wx0 = static_cast<uint32_t>(c & 3);
      if constexpr (QT == kTypeQ6_K) {
        const int hf = c & 1;
        r[u].w1 = u32x4{r[u].w1.x >> (2 * hf), r[u].w1.y >> (2 * hf), r[u].w1.z >> (2 * hf),
                        r[u].w1.w >> (2 * hf)};
      }
    }
  };
  auto commit_stage = [&](int buf, const Raw<QT> *r) {
#pragma unroll
    for (int u = 0; u < kIpt; ++u) commit<QT, AH>(sm, buf, r[u], tid + kT * u);
  };

  // Stage c+1 is converted into the idle buffer and stage c+2 is fetched in
  // every step, branch-free (past the end they repeat the last stage and
  // fill a buffer nobody reads), so that one basic block holds the MFMAs and
  // the conversion and the scheduler can interleave them.
  Raw<QT> raw[kIpt];
  const int c_last = max(c_begin, c_end - 1);
  fetch_stage(raw, c_begin);
  commit_stage(0, raw);
  fetch_stage(raw, min(c_begin + 1, c_last));
  __syncthreads();

  const int arow = wm * kWM + l32;  // + 32 * i
  const int brow = wn * 128 + l32;  // + 32 * j
  for (int c = c_begin; c < c_end; ++c) {
    const int buf = (c - c_begin) & 1;
    const _Float16 *sa = sm.a[buf];
    const _Float16 *sw = sm.w[buf];
#pragma unroll
    for (int ks = 0; ks < kBK / 16; ++ks) {
      h8 fa[kFM], fb[4];
      // rows arow + 32 i (brow + 32 j) share swz(arow) (swz(brow)): period 16
      const int ga = 8 * ((2 * ks + h) ^ swz(arow)), gb = 8 * ((2 * ks + h) ^ swz(brow));
#pragma unroll
      for (int i = 0; i < kFM; ++i)
        fa[i] = *reinterpret_cast<const h8 *>(sa + (arow + 32 * i) * kPitch + ga);
#pragma unroll
      for (int j = 0; j < 4; ++j)
        fb[j] = *reinterpret_cast<const h8 *>(sw + (brow + 32 * j) * kPitch + gb);
#pragma unroll
      for (int i = 0; i < kFM; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(fa[i], fb[j], acc[i][j], 0, 0, 0);
    }
    commit_stage(buf ^ 1, raw);
    fetch_stage(raw, min(c + 2, c_last));
    // issue order: each MFMA followed by a few VALU conversion instructions
#pragma unroll
    for (int i = 0; i < 4 * kFM * 4; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
      __builtin_amdgcn_sched_group_barrier(0x002, IFX_F16_VALU_PER_MFMA, 0);  // VALU
    }
    __syncthreads();
  }

  // Epilogue: lane holds column n and rows 8*(e/4) + 4*h + (e%4) of each tile.
#pragma unroll
  for (int i = 0; i < kFM; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int n = n0 + wn * 128 + 32 * j + l32;
      if (n >= N) continue;
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int m = m0 + wm * kWM + 32 * i + 8 * (e >> 2) + 4 * h + (e & 3);
        if (m >= M) continue;
        const int64_t o = static_cast<int64_t>(m) * N + n;
        float y = acc[i][j][e];
        if constexpr (SPL == 2) {
          static_cast<float *>(Y)[static_cast<int64_t>(split) * M * N + o] = y;
        } else if constexpr (SPL == 1) {
          if (mode == 2 && split == 0) y += static_cast<const float *>(bias)[n];
          atomicAdd(static_cast<float *>(Y) + o, y);
        } else if constexpr (F16OUT) {
          uint16_t *Yh = static_cast<uint16_t *>(Y);
          if (mode == 1) y += h2f(Yh[o]);
          else if (mode == 2) y += h2f(static_cast<const uint16_t *>(bias)[n]);
          Yh[o] = static_cast<uint16_t>(f2h_bits(y));
        } else {
          float *Yf = static_cast<float *>(Y);
          if (mode == 1) y += Yf[o];
          else if (mode == 2) y += static_cast<const float *>(bias)[n];
          Yf[o] = y;
        }
      }
    }
}

// Q8_1 activations -> fp16 in the GEMM's staging order (64 bytes per block),
// once per GEMM instead of once per weight tile, with the conversion the
// GEMM applies itself (i8x4_to_h on the block's fp16 d), so both give the
// same bits.  Thread t writes 16 bytes, words 4q..4q+3 of block t/4
// (q = t%4), i.e. codes 8q..8q+7: consecutive threads store consecutive
// 16-byte chunks.
__global__ __launch_bounds__(256) void k_q8_1_to_f16(const uint8_t *__restrict__ A,
                                                     u32x4 *__restrict__ out, int64_t nchunks) {
  const int64_t t = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (t >= nchunks) return;
  const uint8_t *src = A + (t >> 2) * kQ8_1Bytes;
  const int q = static_cast<int>(t & 3);
  const h2 d = splat(h2f(ldg<uint32_t>(src) & 0xFFFFu));
  const u32x2 c = ldg<u32x2>(src + 4 + 8 * q);
  uint32_t o[4];
  i8x4_to_h(c.x, d, o[0], o[1]);
  i8x4_to_h(c.y, d, o[2], o[3]);
  out[t] = u32x4{o[0], o[1], o[2], o[3]};
}

// The ordered reduction of the SPL = 2 GEMM: y = ((s_0 + s_1) + ...) over
// the splits' slots in split order, then the epilogue (mode 1: + Y, 2:
// + bias[n]).  Four consecutive outputs per thread (16-byte accesses when
// M * N % 4 == 0 and Y is 16-byte aligned).
__global__ __launch_bounds__(256) void k_split_sum(const float *__restrict__ slots,
                                                   float *__restrict__ Y,
                                                   const float *__restrict__ bias, int64_t mn,
                                                   int N, int splits, int mode) {
  const int64_t i = (static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x) * 4;
  if (i >= mn) return;
  if ((mn & 3) == 0 && (reinterpret_cast<uintptr_t>(Y) & 15) == 0) {
    f32x4 t = *reinterpret_cast<const f32x4 *>(slots + i);
    for (int sp = 1; sp < splits; ++sp) t += *reinterpret_cast<const f32x4 *>(slots + sp * mn + i);
    if (mode == 1) t += *reinterpret_cast<const f32x4 *>(Y + i);
    if (mode == 2) {
      const int n = static_cast<int>(i % N);
      t += f32x4{bias[n], bias[(n + 1) % N], bias[(n + 2) % N], bias[(n + 3) % N]};
    }
    *reinterpret_cast<f32x4 *>(Y + i) = t;
    return;
  }
  for (int64_t k = i; k < mn && k < i + 4; ++k) {
    float t = slots[k];
    for (int sp = 1; sp < splits; ++sp) t += slots[sp * mn + k];
    if (mode == 1) t += Y[k];
    if (mode == 2) t += bias[k % N];
    Y[k] = t;
  }
}

namespace {

template <int QT, bool F16OUT, int SPL, bool AH, int WV = IFX_F16_WAVES>
hipError_t launch_k(const uint8_t *W, const uint8_t *A, void *Y, const void *bias, int M, int N,
                    int K, int mode, int m_tiles, int n_tiles, int splits, int cps,
                    hipStream_t s) {
  const void *fn = reinterpret_cast<const void *>(&k_gemm_f16<QT, WV, F16OUT, SPL, AH>);
  // set once per instantiation (a function-local static: thread-safe)
  if (!dry_run()) {
    static const hipError_t attr = hipFuncSetAttribute(
        fn, hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(sizeof(Smem)));
    if (attr != hipSuccess) return attr;
  }
  const dim3 grid(static_cast<unsigned>(m_tiles * n_tiles * splits));
  IFX_LAUNCH(k_gemm_f16, (QT, WV, F16OUT, SPL, AH), grid, dim3(64 * WV), sizeof(Smem), s,
                     W, A, Y, bias, M, N, K, mode, m_tiles, splits, cps);
  return last_error();
}

template <int QT, bool F16OUT, int SPL>
hipError_t launch_a(const uint8_t *W, const uint8_t *A, void *A16, void *Y, const void *bias,
                    int M, int N, int K, int mode, int m_tiles, int n_tiles, int splits, int cps,
                    hipStream_t s) {
  if (!A16)
    return launch_k<QT, F16OUT, SPL, false>(W, A, Y, bias, M, N, K, mode, m_tiles, n_tiles,
                                            splits, cps, s);
  const int64_t nchunks = static_cast<int64_t>(M) * (K >> 5) * 4;
  IFX_LAUNCH0(k_q8_1_to_f16, dim3(static_cast<unsigned>((nchunks + 255) / 256)), dim3(256),
                     0, s, A, static_cast<u32x4 *>(A16), nchunks);
  const hipError_t e = last_error();
  if (e != hipSuccess) return e;
  return launch_k<QT, F16OUT, SPL, true>(W, static_cast<const uint8_t *>(A16), Y, bias, M, N, K,
                                         mode, m_tiles, n_tiles, splits, cps, s);
}

// K splits of a launch: only for fp32 outputs, when the tile grid fills
// less than 3/4 of the 256 CUs (one 512-thread workgroup per CU): as many
// splits as fit in one pass over the CUs, keeping >= 8 stages per workgroup
// (measured, N = 5120, K = 27648, M = 512: 5 splits 273 us, 6 splits 230
// us).  Sets cps (stages per split).
int f16_splits(bool f16, int M, int N, int K, int splits_req, int &cps) {
  const int m_tiles = (M + kBM - 1) / kBM, n_tiles = (N + kBN - 1) / kBN;
  const int nst = K / kBK;
  int splits = 1;
  if (splits_req > 0) {
    splits = splits_req;
  } else if (!f16) {
    const int tiles = m_tiles * n_tiles;
    if (tiles < 192) splits = max(1, min(256 / tiles, nst / 8));
  }
  if (f16) splits = 1;
  if (splits > nst) splits = nst;
  cps = (nst + splits - 1) / splits;
  return (nst + cps - 1) / cps;
}

// slots: NULL, or the ordered reduction's slots (splits x M x N fp32) for a
// launch that splits K.
template <int QT>
hipError_t launch_qt(const uint8_t *W, const uint8_t *A, void *A16, void *Y, const void *bias,
                     bool f16, int M, int N, int K, int mode, int splits_req, float *slots,
                     hipStream_t s) {
  const int m_tiles = (M + kBM - 1) / kBM, n_tiles = (N + kBN - 1) / kBN;
  int cps = 0;
  const int splits = f16_splits(f16, M, N, K, splits_req, cps);
  if (splits > 1 && slots) {
    const hipError_t e = launch_a<QT, false, 2>(W, A, A16, slots, nullptr, M, N, K, mode, m_tiles,
                                                n_tiles, splits, cps, s);
    if (e != hipSuccess) return e;
    const int64_t mn = static_cast<int64_t>(M) * N;
    IFX_LAUNCH0(k_split_sum, dim3(static_cast<unsigned>((mn + 1023) / 1024)), dim3(256), 0, s,
                slots, static_cast<float *>(Y), static_cast<const float *>(bias), mn, N, splits,
                mode);
    return last_error();
  }
  if (splits > 1) {
    if (mode != 1) {  // store / bias: the workgroups add into a zeroed Y
      FillArgs f{};
      f.y[0] = static_cast<float *>(Y);
      f.n[0] = static_cast<int64_t>(M) * N;
      if (launch_fill_zero(f, 1, s) != hipSuccess) return last_error();
    }
    return launch_a<QT, false, 1>(W, A, A16, Y, bias, M, N, K, mode, m_tiles, n_tiles, splits,
                                  cps, s);
  }
  if (f16)
    return launch_a<QT, true, 0>(W, A, A16, Y, bias, M, N, K, mode, m_tiles, n_tiles, 1, cps, s);
  return launch_a<QT, false, 0>(W, A, A16, Y, bias, M, N, K, mode, m_tiles, n_tiles, 1, cps, s);
}

}  // namespace

bool gemm_f16_fits(int qtype, int K) {
  if (qtype == kTypeQ4_K || qtype == kTypeQ6_K) return K % 256 == 0;
  if (qtype == kTypeQ8_0) return K % kBK == 0;
  return false;
}

// Bytes of the fp16 activation copy the GEMM can use (M x K halves), or 0
// when it would not fit the kernel's 32-bit buffer offsets.
int64_t gemm_f16_workspace_bytes(int M, int K) {
  const int64_t b = static_cast<int64_t>(M) * K * 2;
  return b < (int64_t{1} << 32) ? b : 0;
}

// Bytes of the ordered reduction's slots (splits x M x N fp32), or 0 when
// the launch does not split K.
int64_t gemm_f16_slot_bytes(bool f16, int M, int N, int K) {
  int cps = 0;
  const int splits = f16_splits(f16, M, N, K, 0, cps);
  return splits > 1 ? static_cast<int64_t>(splits) * M * N * 4 : 0;
}

// splits_req: 0 = chosen from the tile grid, else forced (tests).  A16:
// caller-owned workspace of gemm_f16_workspace_bytes(M, K) bytes (16-byte
// aligned) for the fp16 activations, converted once before the GEMM; NULL:
// each workgroup converts its Q8_1 activation tiles itself.  Same results.
// slots: NULL (K splits add with fp32 atomics into a zeroed Y), or
// gemm_f16_slot_bytes of 16-byte aligned memory for the ordered reduction.
hipError_t launch_gemm_f16(int qtype, const void *W, const void *A, void *A16, void *Y,
                           const void *bias, bool f16, int M, int N, int K, int mode,
                           int splits_req, hipStream_t stream, float *slots) {
  const uint8_t *w = static_cast<const uint8_t *>(W);
  const uint8_t *a = static_cast<const uint8_t *>(A);
  if (!gemm_f16_fits(qtype, K)) return hipErrorInvalidValue;
  if (A16 && gemm_f16_workspace_bytes(M, K) == 0) A16 = nullptr;
  switch (qtype) {
  case kTypeQ4_K: return launch_qt<kTypeQ4_K>(w, a, A16, Y, bias, f16, M, N, K, mode, splits_req, slots, stream);
  case kTypeQ6_K: return launch_qt<kTypeQ6_K>(w, a, A16, Y, bias, f16, M, N, K, mode, splits_req, slots, stream);
  case kTypeQ8_0: return launch_qt<kTypeQ8_0>(w, a, A16, Y, bias, f16, M, N, K, mode, splits_req, slots, stream);
  default: return hipErrorInvalidValue;
  }
}

// ---------------------------------------------------------------------------
// Static workspace of the no-alloc prefill entry (ifx_qgemm_prefill_noalloc):
// the fp16 activation copy lives in this array instead of caller memory.
// Each GPU holds its own copy, at its own address, until the process ends.
// On the host `scratch` names a host-side stand-in, never a device address:
// host code uses only the address hipGetSymbolAddress returns for the
// current device.
static __device__ __align__(256) uint8_t scratch[IFX_NOALLOC_SCRATCH_BYTES];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void *g_scratch_ptr[kMaxDevices];  // per device, resolved on first use
}  // namespace

// Device address of `scratch` on the current device, resolved once per
// device with that device current.
hipError_t scratch_address(void **out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void *p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return e;
    if (!p) return hipErrorInvalidSymbol;
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return hipSuccess;
}

}  // namespace ifx
