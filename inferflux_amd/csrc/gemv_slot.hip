// gemv_slot.hip -- decode-batch quantized GEMV for 5 <= M <= 8 on the
// gfx950 matrix cores, with weights streamed straight into MFMA operand
// registers: y[m][n] = sum_k W[n][k] * a[m][k], W raw GGUF Q4_K / Q6_K
// blocks, a Q8_1 blocks of 32.
//
// Arithmetic is the reference's MMVQ arithmetic
// (runtime/backends/cuda/native/kernels/mmvq.cuh:49-158 Q4_K, 407-843 Q6_K):
// an exact integer dot per 32-value sub-block (Q6_K: per 16-value group),
// then fp32 scaling by the weight scale and the Q8_1 d; the Q4_K min term
// uses the Q8_1 s = d * sum(q) field.
//
// Batch-row slots.  One v_mfma_i32_32x32x32_i8 multiplies a 32 x 32 tile of
// activation codes (rows) by a 32 x 32 tile of weight codes (K x 32 weight
// rows).  A decode batch has only MP = 8 or 16 rows (M padded), so the 32
// MFMA rows are split into 32 / MP "slots" of MP rows each: in a chain of
// MFMAs accumulating into one result tile, the MFMA of scale block j feeds
// activation codes only to the rows of slot(j) and zeros to the others.
// After the chain, slot s of the result holds the exact integer dot of its
// own block -- several blocks per tile, no padding rows, and no cross-lane
// moves.  Each lane then rescales only real outputs: per lane and block,
// one multiply by the integer weight scale, one convert, one FMA with the
// Q8_1 d (the super-block d is applied once per super-block).
//   Q4_K: block j = 32-value sub-block; slots per chain = 32 / MP.
//   Q6_K: its scales are per 16 values, and the two K halves of an MFMA
//         (lanes 0-31: values 0-15, lanes 32-63: values 16-31 of the block)
//         are the two groups: each group gets a slot of its own.
//
// Lane mapping.  Lane l supplies weight row c = l % 32 of the wave's 32
// rows and K half h = l / 32 of every block: a 16-byte chunk of its row's
// super-block that it loads itself (no LDS for weights; a row's whole
// super-block is in flight in 64 lanes x 5-7 loads).  For the activation
// operand lane l is MFMA row r = l % 32, i.e. batch row r % MP of slot
// r / MP; it loads the 16 codes of its batch row's block for its slot.
// The result layout gives lane l weight row c and batch rows
// {2 (i & ~3) + 4 h + (i & 3)} of each slot.
//
// Work split.  A workgroup owns 32 weight rows and KW waves; wave w walks
// super-blocks w, w + KW, ... with the next one's loads in flight while the
// current one is computed; the KW partial results are summed through LDS.
// Launches with few row groups (N = 2048 has 64) also split the
// super-blocks over gridDim.y workgroups, whose fp32 partial sums are added
// to Y with atomics (Y is zeroed first for the store/bias modes), as the
// reference's atomic fp32 accumulate kernels do (mmvq.cuh:280-401): such
// results are not bitwise reproducible run to run.  fp16 outputs never split.
// The Q8_1 d (and s) of the current super-block go through a 1 KB per-wave
// LDS table, since the rescaling lanes need those of other lanes' rows.
// Grouped launches: up to three projections that share A.
#include "ifx_q8_1.h"

#include <stdlib.h>

namespace ifx {

struct SlotSeg {
  const uint8_t *W;
  void *Y;
  const void *bias;
  int N;
  int blk_begin;
};

struct SlotArgs {
  SlotSeg seg[3];
  int nseg;
  const uint8_t *A;
  int M, K, mode;
  SplitWs ws;  // ordered split: counters per row group, 1 KB slot per (group, split)
  // fused gate/up/SiLU (SW): seg[0] gate, seg[1] up; h = silu(g) * u to H
  // (fp32, fp16 with F16OUT, or none) and its Q8_1 blocks to Q (or none)
  void *H;
  uint8_t *Q;
};

namespace {

// Per (QT, MP): MFMAs per chain (TPC) and chains per super-block (CH).
template <int QT, int MP>
struct SlotGeo {
  static constexpr int kSlots = 32 / MP;
  static constexpr int kTpc = (QT == kTypeQ6_K) ? kSlots / 2 : kSlots;
  static constexpr int kCh = 8 / kTpc;
  static constexpr int kNm = MP / 2;  // batch rows per lane
};

template <int QT>
struct WSb;
template <>
struct WSb<kTypeQ4_K> {
  u32x4 hdr;   // d | dmin, scales[12]
  u32x4 q[4];  // qs[32p + 16h .. +16]: sub-blocks 2p (low), 2p+1 (high)
};
template <>
struct WSb<kTypeQ8_0> {  // tiled rows only
  u32x4 q[8];  // codes 16h .. 16h+15 of blocks 0..7
  u32x4 d;     // the eight blocks' fp16 d
};
template <>
struct WSb<kTypeQ6_K> {
  u32x4 ql[4];  // ql[64 hf + 32 jj + 16h .. +16], index 2 hf + jj
  u32x4 qh[2];  // qh[32 hf + 16h .. +16]
  u32x4 sc;     // scales[16]
  uint32_t d;   // fp16 bits
};

template <int QT, int MP>
struct ASb {
  i32x4 c[SlotGeo<QT, MP>::kCh];  // this lane's codes per chain (zeros if not its slot)
  uint32_t ds[MP / 8];            // d | s of the table entries this lane stages
};

// Q6_K codes minus 32, four per dword: with u the 2 high bits and l the low
// nibble, (16u + l) - 32 = 16 (u - 2) + l, and the top nibble 16 (u - 2)
// mod 256 is 0xE0, 0xF0, 0x00, 0x10 for u = 0..3 -- one byte-select
// (v_perm_b32 with the u bytes as selectors) from that 4-byte table.
__device__ __forceinline__ uint32_t q6_codes(uint32_t l4, uint32_t u2) {
  return __builtin_amdgcn_perm(0u, 0x1000F0E0u, u2) | l4;
}

__device__ __forceinline__ void wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// TL: the tiled layout (ifx_common.h), voff = 16 * (lane % 32) and sb_off
// the tile's byte offset.
template <int QT, bool TL = false>
__device__ __forceinline__ void load_w(WSb<QT> &w, rsrc_t Wr, uint32_t voff, uint32_t sb_off,
                                       int h) {
  static_assert(TL || QT != kTypeQ8_0, "Q8_0 runs on tiled rows only");
  if constexpr (QT == kTypeQ8_0) {
#pragma unroll
    for (int j = 0; j < 8; ++j) w.q[j] = wload<u32x4>(Wr, voff + 1024 * j + 512 * h, sb_off);
    w.d = wload<u32x4>(Wr, voff + 8192, sb_off);
  } else if constexpr (TL && QT == kTypeQ4_K) {
    w.hdr = wload<u32x4>(Wr, voff, sb_off);
#pragma unroll
    for (int p = 0; p < 4; ++p) w.q[p] = wload<u32x4>(Wr, voff + 512 + 1024 * p + 512 * h, sb_off);
  } else if constexpr (TL) {
#pragma unroll
    for (int i = 0; i < 4; ++i) w.ql[i] = wload<u32x4>(Wr, voff + 1024 * i + 512 * h, sb_off);
#pragma unroll
    for (int hf = 0; hf < 2; ++hf) w.qh[hf] = wload<u32x4>(Wr, voff + 4096 + 1024 * hf + 512 * h, sb_off);
    w.sc = wload<u32x4>(Wr, voff + 6144, sb_off);
    w.d = wload<uint16_t>(Wr, 6656 + (voff >> 3), sb_off);
  } else if constexpr (QT == kTypeQ4_K) {
    w.hdr = wload<u32x4>(Wr, voff, sb_off);
#pragma unroll
    for (int p = 0; p < 4; ++p) w.q[p] = wload<u32x4>(Wr, voff + 16 + 32 * p + 16 * h, sb_off);
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i)
      w.ql[i] = wload<u32x4>(Wr, voff + 64 * (i >> 1) + 32 * (i & 1) + 16 * h, sb_off);
#pragma unroll
    for (int hf = 0; hf < 2; ++hf) w.qh[hf] = wload<u32x4>(Wr, voff + 128 + 32 * hf + 16 * h, sb_off);
    w.sc = wload<u32x4>(Wr, voff + 192, sb_off);
    w.d = wload<uint16_t>(Wr, voff + 208, sb_off);
  }
}

// a_off[c]: this lane's code offset for chain c within super-block 0 (or an
// offset past the end of A, which loads zeros); ds_off[u]: table entries.
template <int QT, int MP>
__device__ __forceinline__ void load_a(ASb<QT, MP> &a, rsrc_t Ar, const uint32_t (&a_off)[SlotGeo<QT, MP>::kCh],
                                       const uint32_t (&ds_off)[MP / 8], uint32_t sb_off) {
#pragma unroll
  for (int c = 0; c < SlotGeo<QT, MP>::kCh; ++c) a.c[c] = bload<i32x4>(Ar, a_off[c], sb_off);
#pragma unroll
  for (int u = 0; u < MP / 8; ++u) a.ds[u] = bload<uint32_t>(Ar, ds_off[u], sb_off);
}

__device__ __forceinline__ i32x16 mfma_acc(i32x4 a, i32x4 b, i32x16 c) {
  return __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c, 0, 0, 0);
}

// Weight operand of block j (K half h of this lane) as int8 codes.
template <int QT>
__device__ __forceinline__ i32x4 w_operand(const WSb<QT> &w, int j) {
  if constexpr (QT == kTypeQ8_0) {
    return __builtin_bit_cast(i32x4, w.q[j]);
  } else if constexpr (QT == kTypeQ4_K) {
    const u32x4 q = w.q[j >> 1];
    const int sh = 4 * (j & 1);
    return i32x4{static_cast<int>((q.x >> sh) & 0x0F0F0F0Fu), static_cast<int>((q.y >> sh) & 0x0F0F0F0Fu),
                 static_cast<int>((q.z >> sh) & 0x0F0F0F0Fu), static_cast<int>((q.w >> sh) & 0x0F0F0F0Fu)};
  } else {
    const int hf = j >> 2, jq = j & 3;
    const u32x4 ql = w.ql[2 * hf + (jq & 1)];
    const u32x4 qh = w.qh[hf];
    const int s1 = 4 * (jq >> 1), s2 = 2 * jq;
    auto v = [&](uint32_t l, uint32_t hh) {
      return static_cast<int>(q6_codes((l >> s1) & 0x0F0F0F0Fu, (hh >> s2) & 0x03030303u));
    };
    return i32x4{v(ql.x, qh.x), v(ql.y, qh.y), v(ql.z, qh.z), v(ql.w, qh.w)};
  }
}

}  // namespace

// NP: projections per workgroup (2 for the fused gate/up/SiLU launch).
template <int QT, int MP, int KW, int NP = 1>
constexpr int slot_lds_bytes() {
  constexpr int table = NP * KW * 2 * 8 * MP * 4;                     // per-wave d and s tables
  constexpr int red = NP * (KW > 1 ? KW - 1 : 0) * 64 * (MP / 2) * 4;  // partial results
  constexpr int gu = NP == 2 ? 2 * MP * 32 * 4 : 0;                    // gate/up outputs
  return table + red + gu;
}

// SW: fused gate/up/SiLU (the reference's FusedGateUpSiluGemvQ8_1,
// mmvq.cuh:1686-2030, for decode batches up to 8): a workgroup of 2 KW waves
// owns 32 outputs, waves [0, KW) the gate rows and [KW, 2 KW) the up rows,
// each half exactly as a grouped slot launch of KW waves computes them; then
// one wave forms h = silu(g) * u (the SiLU producer's arithmetic) and
// quantizes each batch row's 32 values into one Q8_1 block, so h and its
// blocks equal grouped GEMV + silu_mul_quantize bit for bit where the
// grouped launch runs the same KW (other KW add the super-blocks' partial
// sums in another order).
// SPLIT: 0 one workgroup per row group; 1 K split over gridDim.y with fp32
// atomics into Y (zeroed first in store / bias mode); 2 K split with the
// ordered reduction through args.ws (split_arrive_last, ifx_common.h);
// 3 as 0, for accumulate and bias launches: the term each output adds (Y
// before the launch, or the bias) is loaded ahead of the weights, so the
// epilogue waits on no dependent load (nothing else writes those outputs
// during the launch: the same bits as 0).
template <int QT, int MP, int KW, bool F16OUT, int SPLIT, bool SW = false, bool TL = false>
__global__ __launch_bounds__(64 * KW * (SW ? 2 : 1)) void k_gemv_slot(const SlotArgs args) {
  using G = SlotGeo<QT, MP>;
  constexpr int NM = G::kNm;
  static_assert(!(SW && SPLIT), "the fused gate/up/SiLU launch does not split K");
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const int bx = blockIdx.x;
  const int wave_all = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int proj = SW ? wave_all / KW : 0;  // SW: 0 gate, 1 up
  const int wave = SW ? wave_all % KW : wave_all;  // wave within its projection
  const int si = SW ? proj
                 : (args.nseg > 2 && bx >= args.seg[2].blk_begin) ? 2
                 : (args.nseg > 1 && bx >= args.seg[1].blk_begin) ? 1 : 0;
  const SlotSeg &sg = args.seg[si];
  const int N = sg.N, M = args.M, K = args.K;
  const int lane = threadIdx.x & 63;
  const int c32 = lane & 31, h = lane >> 5;
  const int n0 = SW ? bx * 32 : (bx - sg.blk_begin) * 32;
  const int nsb = K >> 8;
  constexpr int kSbBytes = (QT == kTypeQ4_K) ? kQ4KBytes : (QT == kTypeQ8_0) ? 8 * kQ8_0Bytes : kQ6KBytes;
  const uint32_t w_row = static_cast<uint32_t>(nsb) * kSbBytes;
  const uint32_t a_row = static_cast<uint32_t>(K >> 5) * kQ8_1Bytes;
  // tiled: whole 32-row groups; tile (group, super-block) at (group * nsb + sb) * kTile
  constexpr int kTile = kTileRows * kSbBytes;
  const rsrc_t Wr = make_rsrc(sg.W, w_row * static_cast<uint32_t>(TL ? (N + 31) & ~31 : N));
  const rsrc_t Ar = make_rsrc(args.A, a_row * static_cast<uint32_t>(M));
  float *dl = reinterpret_cast<float *>(smem) + wave_all * (2 * 8 * MP);  // [8][MP] d
  float *sl = dl + 8 * MP;                                            // [8][MP] s

  const uint32_t w_voff = TL ? 16u * c32 : static_cast<uint32_t>(min(n0 + c32, N - 1)) * w_row;
  const uint32_t w_soff = TL ? static_cast<uint32_t>(n0 / 32) * nsb * kTile : 0u;  // group's first tile
  constexpr int kSbStep = TL ? kTile : kSbBytes;  // bytes between a row's super-blocks
  // activation operand: MFMA row r = c32 = batch row (r % MP) of slot r / MP
  const int am = c32 % MP, aslot = c32 / MP;
  bool a_valid = true;
  int tsel = aslot;  // MFMA within a chain that this lane feeds
  if constexpr (QT == kTypeQ6_K) {
    a_valid = (aslot & 1) == h;
    tsel = aslot >> 1;
  }
  uint32_t a_off[G::kCh];
#pragma unroll
  for (int c = 0; c < G::kCh; ++c) {
    const int j = c * G::kTpc + tsel;
    a_off[c] = a_valid ? static_cast<uint32_t>(am) * a_row + j * kQ8_1Bytes + 4 + 16 * h : kOobOffset;
  }
  uint32_t ds_off[MP / 8];
#pragma unroll
  for (int u = 0; u < MP / 8; ++u) {
    const int e = lane + 64 * u;  // table entry: block e / MP, batch row e % MP
    ds_off[u] = static_cast<uint32_t>(e % MP) * a_row + (e / MP) * kQ8_1Bytes;
  }
  // masks selecting this lane's activation codes for MFMA t of a chain
  uint32_t amask[G::kTpc];
#pragma unroll
  for (int t = 0; t < G::kTpc; ++t) amask[t] = (t == tsel) ? 0xFFFFFFFFu : 0u;

  float acc[NM];
#pragma unroll
  for (int i = 0; i < NM; ++i) acc[i] = 0.0f;

  float early[SPLIT == 3 ? NM : 1];  // SPLIT == 3: the added term, branch-free
  if constexpr (SPLIT == 3) {
    const int nc = min(n0 + c32, N - 1);
    const bool bias_mode = args.mode == 2;
#pragma unroll
    for (int mi = 0; mi < NM; ++mi) {
      const int m = min(2 * (mi & ~3) + 4 * h + (mi & 3), M - 1);
      const int64_t o = static_cast<int64_t>(m) * N + nc;
      const int64_t at = bias_mode ? nc : o;  // no offset from a null bias
      if constexpr (F16OUT)
        early[mi] = h2f(static_cast<const uint16_t *>(bias_mode ? sg.bias : sg.Y)[at]);
      else
        early[mi] = static_cast<const float *>(bias_mode ? sg.bias : sg.Y)[at];
    }
  }

  // this wave's super-blocks: wave index over the split, stride KS * KW
  constexpr bool kSplitK = SPLIT == 1 || SPLIT == 2;
  const int step = kSplitK ? KW * static_cast<int>(gridDim.y) : KW;
  int sb = (kSplitK ? static_cast<int>(blockIdx.y) * KW : 0) + wave;
  WSb<QT> wc;
  ASb<QT, MP> ac;
  if (sb < nsb) {
    load_w<QT, TL>(wc, Wr, w_voff, w_soff + sb * kSbStep, h);
    load_a<QT, MP>(ac, Ar, a_off, ds_off, sb * 8 * kQ8_1Bytes);
  }
  for (; sb < nsb; sb += step) {
    WSb<QT> wn;
    ASb<QT, MP> an;
    const bool more = sb + step < nsb;
    if (more) {
      load_w<QT, TL>(wn, Wr, w_voff, w_soff + (sb + step) * kSbStep, h);
      load_a<QT, MP>(an, Ar, a_off, ds_off, (sb + step) * 8 * kQ8_1Bytes);
    }
    // d and s of this super-block's 8 x MP activation blocks
#pragma unroll
    for (int u = 0; u < MP / 8; ++u) {
      const int e = lane + 64 * u;
      dl[e] = h2f(ac.ds[u] & 0xFFFFu);
      if constexpr (QT == kTypeQ4_K) sl[e] = h2f(ac.ds[u] >> 16);
    }
    wave_sync();

    float part[NM];
#pragma unroll
    for (int i = 0; i < NM; ++i) part[i] = 0.0f;
    if constexpr (QT == kTypeQ4_K) {
      const uint32_t S0 = wc.hdr.y, S1 = wc.hdr.z, S2 = wc.hdr.w;
      // 6-bit scales and mins of sub-blocks 0-3 and 4-7 (quant_common.cuh:83-94)
      const uint64_t sc8 = static_cast<uint64_t>(S0 & 0x3F3F3F3Fu) |
                           (static_cast<uint64_t>((S2 & 0x0F0F0F0Fu) | ((S0 >> 2) & 0x30303030u)) << 32);
      const uint64_t mn8 = static_cast<uint64_t>(S1 & 0x3F3F3F3Fu) |
                           (static_cast<uint64_t>(((S2 >> 4) & 0x0F0F0F0Fu) | ((S1 >> 2) & 0x30303030u)) << 32);
      float pm[NM];
#pragma unroll
      for (int i = 0; i < NM; ++i) pm[i] = 0.0f;
#pragma unroll
      for (int c = 0; c < G::kCh; ++c) {
        i32x16 C = {0};
#pragma unroll
        for (int t = 0; t < G::kTpc; ++t) {
          const int j = c * G::kTpc + t;
          const i32x4 a = ac.c[c] & static_cast<int>(amask[t]);
          C = mfma_acc(a, w_operand<QT>(wc, j), C);
        }
        // result i: slot (8 (i / 4)) / MP -> block j; batch row index mi
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int s = (8 * (i >> 2)) / MP;
          const int j = c * G::kTpc + s;
          const int mi = ((8 * (i >> 2)) % MP) / 2 + (i & 3);
          const int sc = static_cast<int>((sc8 >> (8 * j)) & 0xFFu);
          const float da = dl[j * MP + 2 * (mi & ~3) + 4 * h + (mi & 3)];
          part[mi] += static_cast<float>(__mul24(C[i], sc)) * da;
        }
      }
      // min term: sum_j m_j * s[m][j]
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float fm = static_cast<float>((mn8 >> (8 * j)) & 0xFFu);
#pragma unroll
        for (int mi = 0; mi < NM; ++mi) pm[mi] += sl[j * MP + 2 * (mi & ~3) + 4 * h + (mi & 3)] * fm;
      }
      const float d = h2f(wc.hdr.x & 0xFFFFu), dmin = h2f(wc.hdr.x >> 16);
#pragma unroll
      for (int mi = 0; mi < NM; ++mi) acc[mi] += d * part[mi] - dmin * pm[mi];
    } else if constexpr (QT == kTypeQ8_0) {
      // per block: the exact integer dot times d_w * d_a (mmvq.cuh:886-889)
      const uint32_t dw4[4] = {wc.d.x, wc.d.y, wc.d.z, wc.d.w};
#pragma unroll
      for (int c = 0; c < G::kCh; ++c) {
        i32x16 C = {0};
#pragma unroll
        for (int t = 0; t < G::kTpc; ++t) {
          const int j = c * G::kTpc + t;
          const i32x4 a = ac.c[c] & static_cast<int>(amask[t]);
          C = mfma_acc(a, w_operand<QT>(wc, j), C);
        }
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int s = (8 * (i >> 2)) / MP;
          const int j = c * G::kTpc + s;
          const int mi = ((8 * (i >> 2)) % MP) / 2 + (i & 3);
          const float dw = h2f((dw4[j >> 1] >> (16 * (j & 1))) & 0xFFFFu);
          const float da = dl[j * MP + 2 * (mi & ~3) + 4 * h + (mi & 3)];
          acc[mi] += static_cast<float>(C[i]) * (dw * da);
        }
      }
    } else {
      const uint32_t scw[4] = {wc.sc.x, wc.sc.y, wc.sc.z, wc.sc.w};
#pragma unroll
      for (int c = 0; c < G::kCh; ++c) {
        i32x16 C = {0};
#pragma unroll
        for (int t = 0; t < G::kTpc; ++t) {
          const int j = c * G::kTpc + t;
          const i32x4 a = ac.c[c] & static_cast<int>(amask[t]);
          C = mfma_acc(a, w_operand<QT>(wc, j), C);
        }
        // slot s holds group (block c*TPC + s/2, K half s%2): scale index 2j + s%2
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int s = (8 * (i >> 2)) / MP;
          if (s & 1) continue;  // paired with its odd partner below
          const int j = c * G::kTpc + (s >> 1);
          const int i2 = i + MP / 2;  // same batch row, slot s + 1
          const int mi = ((8 * (i >> 2)) % MP) / 2 + (i & 3);
          const int g = 2 * j;
          const int sc0 = static_cast<int8_t>((scw[g >> 2] >> (8 * (g & 3))) & 0xFFu);
          const int sc1 = static_cast<int8_t>((scw[(g + 1) >> 2] >> (8 * ((g + 1) & 3))) & 0xFFu);
          const float da = dl[j * MP + 2 * (mi & ~3) + 4 * h + (mi & 3)];
          part[mi] += static_cast<float>(__mul24(C[i], sc0) + __mul24(C[i2], sc1)) * da;
        }
      }
      const float d = h2f(wc.d);
#pragma unroll
      for (int mi = 0; mi < NM; ++mi) acc[mi] += d * part[mi];
    }
    wave_sync();  // table reads precede the next super-block's writes
    if (more) {
      wc = wn;
      ac = an;
    }
  }

  constexpr int kNp = SW ? 2 : 1;
  if constexpr (KW > 1) {
    float *red = reinterpret_cast<float *>(smem) + kNp * KW * 2 * 8 * MP +
                 proj * (KW - 1) * NM * 64;  // [KW-1][NM][64] per projection
    if (wave > 0) {
#pragma unroll
      for (int mi = 0; mi < NM; ++mi) red[((wave - 1) * NM + mi) * 64 + lane] = acc[mi];
    }
    __syncthreads();
    if (!SW && SPLIT != 2 && wave > 0) return;
    if (wave == 0) {
#pragma unroll
      for (int w = 0; w < KW - 1; ++w)
#pragma unroll
        for (int mi = 0; mi < NM; ++mi) acc[mi] += red[(w * NM + mi) * 64 + lane];
    }
  }
  if constexpr (SW) {
    // gate/up outputs [projection][batch row][output], then h and Q8_1
    float *gu = reinterpret_cast<float *>(smem) + kNp * KW * 2 * 8 * MP +
                kNp * (KW > 1 ? KW - 1 : 0) * NM * 64;
    if (wave == 0) {
#pragma unroll
      for (int mi = 0; mi < NM; ++mi) {
        const int m = 2 * (mi & ~3) + 4 * h + (mi & 3);
        gu[(proj * MP + m) * 32 + c32] = acc[mi];
      }
    }
    __syncthreads();
    const int m = threadIdx.x >> 3, l = threadIdx.x & 7;  // 8 lanes per batch row
    if (threadIdx.x < 8 * MP && m < M) {
      const f32x4 g4 = *reinterpret_cast<const f32x4 *>(&gu[m * 32 + 4 * l]);
      const f32x4 u4 = *reinterpret_cast<const f32x4 *>(&gu[(MP + m) * 32 + 4 * l]);
      const f32x4 hv = silu_mul4(g4, u4);
      const int64_t o = static_cast<int64_t>(m) * N + n0 + 4 * l;
      if (args.H) {
        if constexpr (F16OUT) {
          const u32x2 hh = {f2h_bits(hv.x) | (f2h_bits(hv.y) << 16),
                            f2h_bits(hv.z) | (f2h_bits(hv.w) << 16)};
          *reinterpret_cast<u32x2 *>(static_cast<uint16_t *>(args.H) + o) = hh;
        } else {
          *reinterpret_cast<f32x4 *>(static_cast<float *>(args.H) + o) = hv;
        }
      }
      if (args.Q)
        quantize4_store(hv.x, hv.y, hv.z, hv.w,
                        args.Q + (static_cast<int64_t>(m) * (N >> 5) + bx) * kQ8_1Bytes, l);
    }
    return;
  }
  float base[NM];  // SPLIT == 2, accumulate mode: Y before this launch
  if constexpr (SPLIT == 2) {
    // wave 0 holds the workgroup's sums (the other waves are done); it alone
    // stores them, counts the workgroup in, and if last reduces the slots
    if (wave > 0) return;
    const int ks = gridDim.y;
    // the accumulate base, requested before the arrival so that its latency
    // overlaps it (only the last workgroup uses it; nothing in this launch
    // writes Y before that workgroup's epilogue)
    const int nc = min(n0 + c32, N - 1);
#pragma unroll
    for (int mi = 0; mi < NM; ++mi) {
      const int m = 2 * (mi & ~3) + 4 * h + (mi & 3);
      base[mi] = (!F16OUT && args.mode == 1 && m < M)
                     ? static_cast<const float *>(sg.Y)[static_cast<int64_t>(m) * N + nc] : 0.0f;
    }
    float *mine = args.ws.part + (static_cast<int64_t>(bx) * ks + blockIdx.y) * 64 * NM + lane;
#pragma unroll
    for (int mi = 0; mi < NM; ++mi)
      if (2 * (mi & ~3) + 4 * h + (mi & 3) < M) st_dev(mine + 64 * mi, acc[mi]);
    wait_own_memory();
    uint32_t prev = 0;
    if (lane == 0)
      prev = __hip_atomic_fetch_add(args.ws.cnt + bx, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (__builtin_amdgcn_readfirstlane(prev) != static_cast<uint32_t>(ks - 1)) return;
    // all slots, this workgroup's included, in split order; eight slots'
    // loads in flight at a time
    const float *slot0 = args.ws.part + static_cast<int64_t>(bx) * ks * 64 * NM + lane;
    float t[NM];
#pragma unroll
    for (int mi = 0; mi < NM; ++mi) t[mi] = 0.0f;
    for (int sp0 = 0; sp0 < ks; sp0 += 8) {
      float v[8][NM];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float *src = slot0 + min(sp0 + j, ks - 1) * 64 * NM;
#pragma unroll
        for (int mi = 0; mi < NM; ++mi) v[j][mi] = ld_dev(src + 64 * mi);
      }
#pragma unroll
      for (int j = 0; j < 8; ++j)
        if (sp0 + j < ks) {
#pragma unroll
          for (int mi = 0; mi < NM; ++mi) t[mi] += v[j][mi];
        }
    }
#pragma unroll
    for (int mi = 0; mi < NM; ++mi) acc[mi] = t[mi];
    split_reset(args.ws.cnt + bx);
  }
  const int n = n0 + c32;
  if (n >= N) return;
  const int mode = args.mode;
#pragma unroll
  for (int mi = 0; mi < NM; ++mi) {
    const int m = 2 * (mi & ~3) + 4 * h + (mi & 3);
    if (m >= M) continue;
    const int64_t o = static_cast<int64_t>(m) * N + n;
    float y = acc[mi];
    if constexpr (SPLIT == 1) {
      // Y was zeroed (store/bias) or holds the accumulate base
      if (mode == 2 && blockIdx.y == 0) y += static_cast<const float *>(sg.bias)[n];
      atomicAdd(static_cast<float *>(sg.Y) + o, y);
    } else if constexpr (SPLIT == 3) {
      if (mode == 1 || mode == 2) y += early[mi];
      if constexpr (F16OUT) static_cast<uint16_t *>(sg.Y)[o] = static_cast<uint16_t>(f2h_bits(y));
      else static_cast<float *>(sg.Y)[o] = y;
    } else if constexpr (F16OUT) {
      uint16_t *Yh = static_cast<uint16_t *>(sg.Y);
      if (mode == 1) y += h2f(Yh[o]);
      else if (mode == 2) y += h2f(static_cast<const uint16_t *>(sg.bias)[n]);
      Yh[o] = static_cast<uint16_t>(f2h_bits(y));
    } else {
      float *Yf = static_cast<float *>(sg.Y);
      if (mode == 1) y += SPLIT == 2 ? base[mi] : Yf[o];
      else if (mode == 2) y += static_cast<const float *>(sg.bias)[n];
      Yf[o] = y;
    }
  }
}

namespace {

// Waves per workgroup and workgroups per row group (the split over
// gridDim.y, fp32 outputs only), measured on MI355X:
//  * wide launches (>= 256 row groups): no split, the fewest waves per
//    workgroup (1..8) that give 4096 waves (an LM head: 1; N = 11008: 8);
//  * few row groups and K up to 24 super-blocks (Q/K/V, O): 8 waves, no
//    split;
//  * few row groups and a longer K (e.g. a down projection with N = 2048):
//    4 waves, 8 splits.
// IFX_SLOT_KW in {1, 2, 4, 8} and IFX_SLOT_SPLIT >= 1 override (tuning;
// read once).  no_split: fp16 outputs without the ordered-split workspace
// (fp16 sums cannot be added with atomics), one workgroup per row group.
void choose_slot_work(int blocks, int nsb, bool no_split, int &kw, int &ks) {
  static const int env_kw = [] {
    const char *e = ifx::tuning_env("IFX_SLOT_KW");
    const int v = e ? atoi(e) : 0;
    return (v == 1 || v == 2 || v == 4 || v == 8) ? v : 0;
  }();
  static const int env_ks = [] {
    const char *e = ifx::tuning_env("IFX_SLOT_SPLIT");
    return e ? atoi(e) : 0;
  }();
  const bool wide = blocks >= 256;
  kw = env_kw;
  if (!kw) {
    // K up to 24 super-blocks: 8 waves, no split (3B O 2048 x 2048 at M = 8,
    // tiled: 4.4 us against 5.8 with 4 waves and 2 ordered splits; 14B Q/K/V
    // 7168 x 5120 at M = 16: 9.8 us against 12.3 with 4 waves and 5 splits)
    kw = wide ? 1 : nsb <= 24 ? 8 : 4;
    while (wide && kw < 8 && blocks * kw < 4096) kw *= 2;
  }
  while (kw > 1 && kw > nsb) kw /= 2;
  ks = env_ks > 0 ? env_ks : (wide || (!env_kw && nsb <= 24)) ? 1 : 8;
  ks = no_split ? 1 : max(1, min(ks, nsb / kw));
}

template <int QT, int MP, int KW, bool F16OUT, int SPLIT, bool TL>
void slot_launch(const SlotArgs &args, int blocks, int ks, hipStream_t s) {
  constexpr int lds = slot_lds_bytes<QT, MP, KW>();
  if constexpr (TL)
    IFX_LAUNCH(k_gemv_slot, (QT, MP, KW, F16OUT, SPLIT, false, true), dim3(blocks, ks),
               dim3(64 * KW), lds, s, args);
  else
    IFX_LAUNCH(k_gemv_slot, (QT, MP, KW, F16OUT, SPLIT), dim3(blocks, ks), dim3(64 * KW), lds,
               s, args);
}

template <int QT, int MP, int KW, bool TL>
void slot_split(const SlotArgs &args, int blocks, int ks, bool f16, hipStream_t s) {
  const bool adds = args.mode != 0;  // accumulate / bias: the term loaded early
  if (f16) {  // a split fp16 launch is ordered (choose_slot_work)
    if (ks > 1) slot_launch<QT, MP, KW, true, 2, TL>(args, blocks, ks, s);
    else if (adds) slot_launch<QT, MP, KW, true, 3, TL>(args, blocks, 1, s);
    else slot_launch<QT, MP, KW, true, 0, TL>(args, blocks, 1, s);
  } else if (ks == 1) {
    if (adds) slot_launch<QT, MP, KW, false, 3, TL>(args, blocks, 1, s);
    else slot_launch<QT, MP, KW, false, 0, TL>(args, blocks, 1, s);
  } else if (args.ws.cnt) {
    slot_launch<QT, MP, KW, false, 2, TL>(args, blocks, ks, s);
  } else {
    if (args.mode != 1) {  // store / bias: the splits add into zeroed outputs
      FillArgs f{};
      for (int i = 0; i < args.nseg; ++i) {
        f.y[i] = static_cast<float *>(args.seg[i].Y);
        f.n[i] = static_cast<int64_t>(args.M) * args.seg[i].N;
      }
      // a failed fill stays set for the caller's hipGetLastError
      if (launch_fill_zero(f, args.nseg, s) != hipSuccess) return;
    }
    slot_launch<QT, MP, KW, false, 1, TL>(args, blocks, ks, s);
  }
}

template <int QT, int MP, bool TL>
void slot_kw(const SlotArgs &args, int blocks, bool f16, hipStream_t s) {
  int kw = 8, ks = 1;
  choose_slot_work(blocks, args.K >> 8, f16 && !args.ws.cnt, kw, ks);
  switch (kw) {
  case 1: slot_split<QT, MP, 1, TL>(args, blocks, ks, f16, s); break;
  case 2: slot_split<QT, MP, 2, TL>(args, blocks, ks, f16, s); break;
  case 4: slot_split<QT, MP, 4, TL>(args, blocks, ks, f16, s); break;
  default: slot_split<QT, MP, 8, TL>(args, blocks, ks, f16, s); break;
  }
}

// MP = 16 (two slots) is instantiable but measured slower than the
// LDS-staged MFMA kernel for 9 <= M <= 16 (twice the rescale work per lane
// at 2-3 waves per SIMD), so only M <= 8 is routed here.
template <int QT, bool TL>
void slot_q(const SlotArgs &args, int blocks, bool f16, hipStream_t s) {
  if (TL && args.M > 8) slot_kw<QT, 16, TL>(args, blocks, f16, s);
  else slot_kw<QT, 8, TL>(args, blocks, f16, s);
}

}  // namespace

// The fused gate/up/SiLU launch: 4 waves per projection and workgroup, no
// K split (one workgroup per 32 outputs).  Measured on MI355X against 1, 2
// and 8 waves (3B gate/up 11008 x 2048 at M = 3 / 4 / 8: 10.9 / 10.9 / 11.7 us
// against 12.4 / 12.4 / 13.1 with 8; 14B 13824 x 5120 at M = 8: 24.4 against
// 27.1).  With fewer than 4 super-blocks per row the waves match them.
// IFX_SLOT_KW overrides, as for the plain launch.
template <int QT, int MP, int KW, bool TL>
void slot_swiglu_launch(const SlotArgs &args, bool f16h, hipStream_t s) {
  constexpr int lds = slot_lds_bytes<QT, MP, KW, 2>();
  const dim3 grid(args.seg[0].N / 32);
  if constexpr (TL) {
    if (f16h) IFX_LAUNCH(k_gemv_slot, (QT, MP, KW, true, false, true, true), grid, dim3(128 * KW), lds, s, args);
    else IFX_LAUNCH(k_gemv_slot, (QT, MP, KW, false, false, true, true), grid, dim3(128 * KW), lds, s, args);
  } else {
    if (f16h) IFX_LAUNCH(k_gemv_slot, (QT, MP, KW, true, false, true), grid, dim3(128 * KW), lds, s, args);
    else IFX_LAUNCH(k_gemv_slot, (QT, MP, KW, false, false, true), grid, dim3(128 * KW), lds, s, args);
  }
}

template <int QT, bool TL>
void slot_swiglu_q(const SlotArgs &args, bool f16h, hipStream_t s) {
  int kw = 4, ks = 1;
  if (ifx::tuning_env("IFX_SLOT_KW")) choose_slot_work(1 << 20, args.K >> 8, false, kw, ks);
  while (kw > 1 && kw > (args.K >> 8)) kw /= 2;
  // tiled rows above M = 8: two 16-row slots per MFMA
  if (TL && args.M > 8) {
    switch (kw) {
    case 1: slot_swiglu_launch<QT, 16, 1, TL>(args, f16h, s); break;
    case 2: slot_swiglu_launch<QT, 16, 2, TL>(args, f16h, s); break;
    case 4: slot_swiglu_launch<QT, 16, 4, TL>(args, f16h, s); break;
    default: slot_swiglu_launch<QT, 16, 8, TL>(args, f16h, s); break;
    }
    return;
  }
  switch (kw) {
  case 1: slot_swiglu_launch<QT, 8, 1, TL>(args, f16h, s); break;
  case 2: slot_swiglu_launch<QT, 8, 2, TL>(args, f16h, s); break;
  case 4: slot_swiglu_launch<QT, 8, 4, TL>(args, f16h, s); break;
  default: slot_swiglu_launch<QT, 8, 8, TL>(args, f16h, s); break;
  }
}

bool gemv_slot_fits(int qtype, int M, int K) {
  const bool t = qtype == kTypeQ4_KT || qtype == kTypeQ6_KT || qtype == kTypeQ8_0T;
  return (qtype == kTypeQ4_K || qtype == kTypeQ6_K || t) && M >= 1 && M <= (t ? 16 : 8) &&
         K % 256 == 0 && K > 0;
}

// count projections (1..3) share A; geometry checked by the caller
// (gemv_slot_fits, 32-bit byte ranges).
// Workspace bytes of the ordered split (0: the launch does not split):
// counters (256-byte aligned) then one 1 KB slot per (row group, split).
int64_t gemv_slot_workspace_bytes(int count, const int *N, bool f16, int M, int K) {
  int blocks = 0;
  for (int i = 0; i < count; ++i) blocks += (N[i] + 31) / 32;
  int kw = 8, ks = 1;
  (void)f16;  // fp16 outputs split as fp32 ones when the workspace is given
  choose_slot_work(blocks, K >> 8, false, kw, ks);
  if (ks <= 1) return 0;
  const int nm = M > 8 ? 8 : 4;  // fp32 sums per lane (MP / 2)
  return (static_cast<int64_t>(blocks) * 4 + 255) / 256 * 256 +
         static_cast<int64_t>(blocks) * ks * 64 * nm * 4;
}

// ws: the ordered-split workspace (gemv_slot_workspace_bytes, counters
// zero), or nullptr for atomics.
hipError_t launch_gemv_slot(int qtype, int count, const void *const *W, void *const *Y,
                            const int *N, const void *bias, const void *A, bool f16, int M, int K,
                            int mode, hipStream_t stream, void *ws) {
  if (!gemv_slot_fits(qtype, M, K) || count < 1 || count > 3) return hipErrorInvalidValue;
  SlotArgs args{};
  int blocks = 0;
  for (int i = 0; i < count; ++i) {
    args.seg[i] = SlotSeg{static_cast<const uint8_t *>(W[i]), Y[i], i == 0 ? bias : nullptr, N[i], blocks};
    blocks += (N[i] + 31) / 32;
  }
  if (ws) {
    args.ws.cnt = static_cast<uint32_t *>(ws);
    args.ws.part = reinterpret_cast<float *>(static_cast<uint8_t *>(ws) +
                                             (static_cast<int64_t>(blocks) * 4 + 255) / 256 * 256);
  }
  args.nseg = count;
  args.A = static_cast<const uint8_t *>(A);
  args.M = M;
  args.K = K;
  args.mode = mode;
  switch (qtype) {
  case kTypeQ4_K: slot_q<kTypeQ4_K, false>(args, blocks, f16, stream); break;
  case kTypeQ6_K: slot_q<kTypeQ6_K, false>(args, blocks, f16, stream); break;
  case kTypeQ4_KT: slot_q<kTypeQ4_K, true>(args, blocks, f16, stream); break;
  case kTypeQ8_0T: slot_q<kTypeQ8_0, true>(args, blocks, f16, stream); break;
  default: slot_q<kTypeQ6_K, true>(args, blocks, f16, stream); break;
  }
  return last_error();
}

// Fused gate/up/SiLU for 1 <= M <= 8, tiled rows up to M = 16 (K % 256 == 0, N % 32 == 0;
// checked by the caller): H (fp32 / fp16 with f16h, or NULL) and / or the
// Q8_1 blocks Q (or NULL).
hipError_t launch_gemv_slot_swiglu(int qtype, const void *Wg, const void *Wu, const void *A,
                                   void *H, bool f16h, void *Q, int M, int N, int K,
                                   hipStream_t stream) {
  const bool t = qtype == kTypeQ4_KT || qtype == kTypeQ6_KT || qtype == kTypeQ8_0T;
  if (!gemv_slot_fits(qtype, M, K) || M > (t ? 16 : 8) || N % 32 != 0) return hipErrorInvalidValue;
  SlotArgs args{};
  args.seg[0] = SlotSeg{static_cast<const uint8_t *>(Wg), nullptr, nullptr, N, 0};
  args.seg[1] = SlotSeg{static_cast<const uint8_t *>(Wu), nullptr, nullptr, N, 0};
  args.nseg = 2;
  args.A = static_cast<const uint8_t *>(A);
  args.M = M;
  args.K = K;
  args.mode = 0;
  args.H = H;
  args.Q = static_cast<uint8_t *>(Q);
  switch (qtype) {
  case kTypeQ4_K: slot_swiglu_q<kTypeQ4_K, false>(args, f16h, stream); break;
  case kTypeQ6_K: slot_swiglu_q<kTypeQ6_K, false>(args, f16h, stream); break;
  case kTypeQ4_KT: slot_swiglu_q<kTypeQ4_K, true>(args, f16h, stream); break;
  case kTypeQ8_0T: slot_swiglu_q<kTypeQ8_0, true>(args, f16h, stream); break;
  default: slot_swiglu_q<kTypeQ6_K, true>(args, f16h, stream); break;
  }
  return last_error();
}

}  // namespace ifx
