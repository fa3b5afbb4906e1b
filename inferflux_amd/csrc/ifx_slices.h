// ifx_slices.h -- the per-lane slice arithmetic of the weight-streaming
// GEMV (gemv.hip): a lane's
// weight bytes of one slice of a row, the matching Q8_1 activation codes
// and scales, and the integer dot plus fp32 scaling of
// runtime/backends/cuda/native/kernels/mmvq.cuh:62-127 (Q4_K), 424-474
// (Q6_K), with the Q4_K min term from the Q8_1 s field (mmvq.cuh:121-125).
// Every form of that GEMV (plain, grouped, fused producers, SiLU epilogue)
// uses this one definition, so their row sums are formed by the same
// instructions in the same order.
#pragma once

#include "ifx_q8_1.h"

namespace ifx {
enum OutMode { kOutStore = 0, kOutAccum = 1, kOutBias = 2 };


// ---------------------------------------------------------------------------
// Q4_K: slice j (0..7) of super-block b covers qs bytes 16j..16j+15, i.e.
// values 16h..16h+15 (h = j & 1) of sub-blocks 2p (low nibbles) and 2p+1
// (high nibbles), p = j >> 1.
// ---------------------------------------------------------------------------
// Q5 = true: Q5_K (same header and qs as Q4_K, qs at +48, and qh[32] at +16
// whose bit j of byte e is the fifth bit of value e of sub-block j); the
// lane also loads qh bytes 16h..16h+15 and ORs the bits in as bit 4 of each
// code (codes 0..31).
template <int MC, int R, bool Q5 = false>
__device__ __forceinline__ void q4k_slice(const rsrc_t (&Wr)[R], rsrc_t Ar, const uint32_t (&rows)[R],
                                          uint32_t a_row, int mvalid, int s, float (&acc)[R][MC]) {
  const int b = s >> 3, j = s & 7, p = j >> 1, h = j & 1;
  // weights first: all R rows in flight before anything waits.  rows[r] is
  // the wave-uniform byte offset of row r; the lane adds its block offset.
  u32x4 hdr[R], q[R], qh[R];
  const uint32_t wo = b * (Q5 ? kQ5KBytes : kQ4KBytes);
#pragma unroll
  for (int r = 0; r < R; ++r) {
    // the 16-byte header is loaded by one lane of the eight that share the
    // super-block (lane & 7 == 0, i.e. j == 0) and broadcast to the others
    hdr[r] = u32x4{0, 0, 0, 0};
    if (j == 0) hdr[r] = wload<u32x4>(Wr[r], wo, rows[r]);
    q[r] = wload<u32x4>(Wr[r], wo + (Q5 ? 48 : 16) + 16 * j, rows[r]);
    if constexpr (Q5) qh[r] = wload<u32x4>(Wr[r], wo + 16 + 16 * h, rows[r]);
  }
  // activations: Q8_1 blocks (b*8 + 2p) and (b*8 + 2p + 1), bytes 16h..16h+15
  i32x4 xa[MC], xb[MC];
  float da[MC], db[MC], sa[MC], sbv[MC];
#pragma unroll
  for (int c = 0; c < MC; ++c) {
    if (c == 0 || c < mvalid) {  // mvalid >= 1
      const uint32_t ao = (b * 8 + 2 * p) * kQ8_1Bytes;
      const uint32_t dsa = bload<uint32_t>(Ar, ao, c * a_row);
      const uint32_t dsb = bload<uint32_t>(Ar, ao + kQ8_1Bytes, c * a_row);
      xa[c] = bload<i32x4>(Ar, ao + 4 + 16 * h, c * a_row);
      xb[c] = bload<i32x4>(Ar, ao + kQ8_1Bytes + 4 + 16 * h, c * a_row);
      da[c] = h2f(dsa & 0xFFFFu);
      db[c] = h2f(dsb & 0xFFFFu);
      // the min term is per 32-value sub-block: only the h == 0 lane adds it
      sa[c] = h ? 0.0f : h2f(dsa >> 16);
      sbv[c] = h ? 0.0f : h2f(dsb >> 16);
    } else {
      xa[c] = xb[c] = i32x4{0, 0, 0, 0};
      da[c] = db[c] = sa[c] = sbv[c] = 0.0f;
    }
  }
  const int shift = 8 * ((2 * p) & 3);
  const uint32_t lo_mask = p < 2 ? 0x3F3F3F3Fu : 0x0F0F0F0Fu;
  const uint32_t top_mask = p < 2 ? 0u : 0x30303030u;
#pragma unroll
  for (int r = 0; r < R; ++r)
    hdr[r] = u32x4{bcast8(hdr[r].x), bcast8(hdr[r].y), bcast8(hdr[r].z), bcast8(hdr[r].w)};
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const float d = h2f(hdr[r].x & 0xFFFFu);
    const float dmin = h2f(hdr[r].x >> 16);
    // 6-bit scale/min unpack (quant_common.cuh:83-94) for 4 sub-blocks per
    // dword: sub-blocks 0-3 from bytes 0-7, 4-7 from bytes 8-11 + top bits.
    // Branch-free: the low bits come from S0/S1 (p < 2, six bits) or from
    // the nibbles of S2 (p >= 2, plus the top two bits of S0/S1); the
    // masks are per-lane constants.
    const uint32_t S0 = hdr[r].y, S1 = hdr[r].z, S2 = hdr[r].w;
    const uint32_t scw = ((p < 2 ? S0 : S2) & lo_mask) | ((S0 >> 2) & top_mask);
    const uint32_t mw = ((p < 2 ? S1 : (S2 >> 4)) & lo_mask) | ((S1 >> 2) & top_mask);
    const uint32_t sct = scw >> shift, mt = mw >> shift;
    const float dsc0 = d * static_cast<float>(sct & 0xFFu);
    const float dsc1 = d * static_cast<float>((sct >> 8) & 0xFFu);
    const float dm0 = dmin * static_cast<float>(mt & 0xFFu);
    const float dm1 = dmin * static_cast<float>((mt >> 8) & 0xFFu);
    int lo0 = q[r].x & 0x0F0F0F0F, hi0 = (q[r].x >> 4) & 0x0F0F0F0F;
    int lo1 = q[r].y & 0x0F0F0F0F, hi1 = (q[r].y >> 4) & 0x0F0F0F0F;
    int lo2 = q[r].z & 0x0F0F0F0F, hi2 = (q[r].z >> 4) & 0x0F0F0F0F;
    int lo3 = q[r].w & 0x0F0F0F0F, hi3 = (q[r].w >> 4) & 0x0F0F0F0F;
    if constexpr (Q5) {
      // bit 2p of qh -> sub-block 2p (low nibbles), bit 2p+1 -> 2p+1
      const int sl = 2 * p, sh5 = 2 * p + 1;
      lo0 |= ((qh[r].x >> sl) & 0x01010101u) << 4;
      lo1 |= ((qh[r].y >> sl) & 0x01010101u) << 4;
      lo2 |= ((qh[r].z >> sl) & 0x01010101u) << 4;
      lo3 |= ((qh[r].w >> sl) & 0x01010101u) << 4;
      hi0 |= ((qh[r].x >> sh5) & 0x01010101u) << 4;
      hi1 |= ((qh[r].y >> sh5) & 0x01010101u) << 4;
      hi2 |= ((qh[r].z >> sh5) & 0x01010101u) << 4;
      hi3 |= ((qh[r].w >> sh5) & 0x01010101u) << 4;
    }
#pragma unroll
    for (int c = 0; c < MC; ++c) {
      int dl = dot4(lo0, xa[c].x, 0);
      dl = dot4(lo1, xa[c].y, dl);
      dl = dot4(lo2, xa[c].z, dl);
      dl = dot4(lo3, xa[c].w, dl);
      int dh = dot4(hi0, xb[c].x, 0);
      dh = dot4(hi1, xb[c].y, dh);
      dh = dot4(hi2, xb[c].z, dh);
      dh = dot4(hi3, xb[c].w, dh);
      acc[r][c] += dsc0 * da[c] * static_cast<float>(dl) + dsc1 * db[c] * static_cast<float>(dh) -
                   (dm0 * sa[c] + dm1 * sbv[c]);
    }
  }
}

// ---------------------------------------------------------------------------
// Q4_K, wide slices (MC <= 2): slice w (0..3) of super-block b covers qs
// bytes 32w..32w+31, i.e. all 32 values of sub-blocks 2w (low nibbles) and
// 2w+1 (high nibbles).  One lane per 64 weights: the header broadcast, the
// 6-bit scale/min decode and the min term are paid once per 32 bytes
// instead of once per 16 (the GEMV is VALU co-limited at M <= 2).  The row
// of load r is at voff[r] + soff[r] (one of the two is zero: per-lane rows
// in half-wave mode, wave-uniform rows otherwise).
// ---------------------------------------------------------------------------
// Activation sources of the slice functions: the caller's Q8_1 tensor
// (buffer loads) or a copy of it in LDS (the GEMV with a fused RMSNorm).
struct AGlobal {
  rsrc_t r;
  uint32_t a_row;
  template <typename T>
  __device__ __forceinline__ T get(uint32_t o, int c) const {
    return bload<T>(r, o, c * a_row);
  }
};
// The caller's Q8_1 tensor written earlier in the same launch by other
// workgroups: device-coherent buffer loads (cache policy sc1).
struct AGlobalDev {
  rsrc_t r;
  uint32_t a_row;
  template <typename T>
  __device__ __forceinline__ T get(uint32_t o, int c) const {
    constexpr int kSc1 = 0x10;
    if constexpr (sizeof(T) == 16)
      return __builtin_bit_cast(T, __builtin_amdgcn_raw_buffer_load_b128(r, o, c * a_row, kSc1));
    else if constexpr (sizeof(T) == 4)
      return __builtin_bit_cast(T, __builtin_amdgcn_raw_buffer_load_b32(r, o, c * a_row, kSc1));
    else
      return __builtin_bit_cast(T, __builtin_amdgcn_raw_buffer_load_b16(r, o, c * a_row, kSc1));
  }
};
struct ALds {
  const uint8_t *p;
  uint32_t a_row;
  template <typename T>
  __device__ __forceinline__ T get(uint32_t o, int c) const {
    return ldg<T>(p + c * a_row + o);
  }
};

// Q8_1 activations in LDS in the split layout of ifx_q8_1.h (split_codes,
// split_ds): per batch column `stride` bytes.
struct ALdsS {
  const uint8_t *p;
  uint32_t stride;
  uint32_t ds0;  // offset of the d | s words in a column: 80 K / 64
};
template <typename AS>
inline constexpr bool kSplitA = false;
template <>
inline constexpr bool kSplitA<ALdsS> = true;

// The weight bytes of wide slice s of R rows, loaded before their use.
template <int R>
struct Q4Wide {
  u32x4 hdr[R], q0[R], q1[R];
};

template <int R>
__device__ __forceinline__ void q4k_wide_load(Q4Wide<R> &wt, const rsrc_t Wr,
                                              const uint32_t (&voff)[R], const uint32_t (&soff)[R],
                                              int s) {
  const int b = s >> 2, w = s & 3;
  const uint32_t wo = b * kQ4KBytes;
#pragma unroll
  for (int r = 0; r < R; ++r) {
    // header: every lane loads its super-block's 16-byte header itself (no
    // branch, no broadcast; the four lanes' requests hit the same line)
    wt.hdr[r] = wload<u32x4>(Wr, voff[r] + wo, soff[r]);
    wt.q0[r] = wload<u32x4>(Wr, voff[r] + wo + 16 + 32 * w, soff[r]);
    wt.q1[r] = wload<u32x4>(Wr, voff[r] + wo + 32 + 32 * w, soff[r]);
  }
}

template <int MC, int R, typename AS>
__device__ __forceinline__ void q4k_wide_compute(const Q4Wide<R> &wt, const AS &as, int mvalid,
                                                 int s, float (&acc)[R][MC]) {
  const int b = s >> 2, w = s & 3;
  // activations: Q8_1 blocks 8b + 2w and 8b + 2w + 1, all 32 codes of each
  i32x4 xa0[MC], xa1[MC], xb0[MC], xb1[MC];
  float da[MC], db[MC], sa[MC], sbv[MC];
#pragma unroll
  for (int c = 0; c < MC; ++c) {
    if (c == 0 || c < mvalid) {  // mvalid >= 1
      uint32_t dsa, dsb;
      if constexpr (kSplitA<AS>) {
        // blocks 8b + 2w and + 1: one 80-byte slot, one 8-byte d | s pair
        const uint8_t *col = as.p + c * as.stride;
        const uint8_t *q = col + (b * 4 + w) * 80;
        const u32x2 ds2 = ldg<u32x2>(col + as.ds0 + (b * 8 + 2 * w) * 4);
        dsa = ds2.x;
        dsb = ds2.y;
        xa0[c] = ldg<i32x4>(q);
        xa1[c] = ldg<i32x4>(q + 16);
        xb0[c] = ldg<i32x4>(q + 32);
        xb1[c] = ldg<i32x4>(q + 48);
      } else {
        const uint32_t ao = (b * 8 + 2 * w) * kQ8_1Bytes;
        dsa = as.template get<uint32_t>(ao, c);
        dsb = as.template get<uint32_t>(ao + kQ8_1Bytes, c);
        xa0[c] = as.template get<i32x4>(ao + 4, c);
        xa1[c] = as.template get<i32x4>(ao + 20, c);
        xb0[c] = as.template get<i32x4>(ao + kQ8_1Bytes + 4, c);
        xb1[c] = as.template get<i32x4>(ao + kQ8_1Bytes + 20, c);
      }
      da[c] = h2f(dsa & 0xFFFFu);
      db[c] = h2f(dsb & 0xFFFFu);
      sa[c] = h2f(dsa >> 16);
      sbv[c] = h2f(dsb >> 16);
    } else {
      xa0[c] = xa1[c] = xb0[c] = xb1[c] = i32x4{0, 0, 0, 0};
      da[c] = db[c] = sa[c] = sbv[c] = 0.0f;
    }
  }
  const int shift = 8 * ((2 * w) & 3);
  const uint32_t lo_mask = w < 2 ? 0x3F3F3F3Fu : 0x0F0F0F0Fu;
  const uint32_t top_mask = w < 2 ? 0u : 0x30303030u;
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const float d = h2f(wt.hdr[r].x & 0xFFFFu);
    const float dmin = h2f(wt.hdr[r].x >> 16);
    // 6-bit scale/min unpack (quant_common.cuh:83-94), branch-free
    const uint32_t S0 = wt.hdr[r].y, S1 = wt.hdr[r].z, S2 = wt.hdr[r].w;
    const uint32_t scw = ((w < 2 ? S0 : S2) & lo_mask) | ((S0 >> 2) & top_mask);
    const uint32_t mw = ((w < 2 ? S1 : (S2 >> 4)) & lo_mask) | ((S1 >> 2) & top_mask);
    const uint32_t sct = scw >> shift, mt = mw >> shift;
    const float dsc0 = d * static_cast<float>(sct & 0xFFu);
    const float dsc1 = d * static_cast<float>((sct >> 8) & 0xFFu);
    const float dm0 = dmin * static_cast<float>(mt & 0xFFu);
    const float dm1 = dmin * static_cast<float>((mt >> 8) & 0xFFu);
    const uint32_t qv[8] = {wt.q0[r].x, wt.q0[r].y, wt.q0[r].z, wt.q0[r].w,
                            wt.q1[r].x, wt.q1[r].y, wt.q1[r].z, wt.q1[r].w};
#pragma unroll
    for (int c = 0; c < MC; ++c) {
      const int xa[8] = {xa0[c].x, xa0[c].y, xa0[c].z, xa0[c].w, xa1[c].x, xa1[c].y, xa1[c].z, xa1[c].w};
      const int xb[8] = {xb0[c].x, xb0[c].y, xb0[c].z, xb0[c].w, xb1[c].x, xb1[c].y, xb1[c].z, xb1[c].w};
      int dl = 0, dh = 0;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        dl = dot4(static_cast<int>(qv[i] & 0x0F0F0F0Fu), xa[i], dl);
        dh = dot4(static_cast<int>((qv[i] >> 4) & 0x0F0F0F0Fu), xb[i], dh);
      }
      acc[r][c] += dsc0 * da[c] * static_cast<float>(dl) + dsc1 * db[c] * static_cast<float>(dh) -
                   (dm0 * sa[c] + dm1 * sbv[c]);
    }
  }
}

template <int MC, int R>
__device__ __forceinline__ void q4k_wide(const rsrc_t Wr, rsrc_t Ar, const uint32_t (&voff)[R],
                                         const uint32_t (&soff)[R], uint32_t a_row, int mvalid,
                                         int s, float (&acc)[R][MC]) {
  Q4Wide<R> wt;
  q4k_wide_load<R>(wt, Wr, voff, soff, s);
  q4k_wide_compute<MC, R>(wt, AGlobal{Ar, a_row}, mvalid, s, acc);
}

// ---------------------------------------------------------------------------
// Q6_K: slice j of super-block b: group g = j >> 2, ql half cc = (j >> 1) & 1
// (sub-blocks cc and cc + 2), values 16h..16h+15 (h = j & 1).
// ---------------------------------------------------------------------------
// RS: the row-split Q6_K_R layout of a row of K values (ifx_common.h).
template <int MC, int R, bool RS = false>
__device__ __forceinline__ void q6k_slice(const rsrc_t (&Wr)[R], rsrc_t Ar, const uint32_t (&rows)[R],
                                          uint32_t a_row, int mvalid, int s, float (&acc)[R][MC],
                                          int K = 0) {
  const int b = s >> 3, j = s & 7, g = j >> 2, cc = (j >> 1) & 1, h = j & 1;
  u32x4 ql[R], qh[R];
  u32x2 scw[R];
  uint16_t dbits[R];
  const uint32_t wo = b * kQ6KBytes;
  const uint32_t qh0 = K >> 1, sc0 = qh0 + (K >> 2), d0 = sc0 + (K >> 4);
  const uint32_t o_ql = RS ? b * 128 + g * 64 + cc * 32 + 16 * h : wo + g * 64 + cc * 32 + 16 * h;
  const uint32_t o_qh = RS ? qh0 + b * 64 + g * 32 + 16 * h : wo + 128 + g * 32 + 16 * h;
  const uint32_t o_sc = RS ? sc0 + b * 16 + g * 8 : wo + 192 + g * 8;
  const uint32_t o_d = RS ? d0 + b * 2 : wo + 208;
#pragma unroll
  for (int r = 0; r < R; ++r) {
    ql[r] = wload<u32x4>(Wr[r], o_ql, rows[r]);
    qh[r] = wload<u32x4>(Wr[r], o_qh, rows[r]);
    scw[r] = wload<u32x2>(Wr[r], o_sc, rows[r]);
    dbits[r] = wload<uint16_t>(Wr[r], o_d, rows[r]);
  }
  i32x4 xa[MC], xb[MC];
  float da[MC], db[MC];
  int suma[MC], sumb[MC];
#pragma unroll
  for (int c = 0; c < MC; ++c) {
    if (c == 0 || c < mvalid) {  // mvalid >= 1
      const uint32_t ao = (b * 8 + g * 4 + cc) * kQ8_1Bytes, bo = ao + 2 * kQ8_1Bytes;
      xa[c] = bload<i32x4>(Ar, ao + 4 + 16 * h, c * a_row);
      xb[c] = bload<i32x4>(Ar, bo + 4 + 16 * h, c * a_row);
      da[c] = h2f(bload<uint16_t>(Ar, ao, c * a_row));
      db[c] = h2f(bload<uint16_t>(Ar, bo, c * a_row));
      // 32 * sum of the activation codes: the -32 offset of Q6_K codes
      int s0 = dot4(0x01010101, xa[c].x, 0);
      s0 = dot4(0x01010101, xa[c].y, s0);
      s0 = dot4(0x01010101, xa[c].z, s0);
      s0 = dot4(0x01010101, xa[c].w, s0);
      int s1 = dot4(0x01010101, xb[c].x, 0);
      s1 = dot4(0x01010101, xb[c].y, s1);
      s1 = dot4(0x01010101, xb[c].z, s1);
      s1 = dot4(0x01010101, xb[c].w, s1);
      suma[c] = 32 * s0;
      sumb[c] = 32 * s1;
    } else {
      xa[c] = xb[c] = i32x4{0, 0, 0, 0};
      da[c] = db[c] = 0.0f;
      suma[c] = sumb[c] = 0;
    }
  }
  const int sh_a = 2 * cc, sh_b = 2 * cc + 4, scs = 8 * (2 * cc + h);
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const float d = h2f(dbits[r]);
    // scales[g*8 + 2*sub + h] for sub = cc (dword 0) and sub = cc + 2 (dword 1)
    const float dsa = d * static_cast<float>(static_cast<int8_t>((scw[r].x >> scs) & 0xFFu));
    const float dsb = d * static_cast<float>(static_cast<int8_t>((scw[r].y >> scs) & 0xFFu));
    const uint32_t qlv[4] = {ql[r].x, ql[r].y, ql[r].z, ql[r].w};
    const uint32_t qhv[4] = {qh[r].x, qh[r].y, qh[r].z, qh[r].w};
    int va[4], vb[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      va[i] = static_cast<int>((qlv[i] & 0x0F0F0F0Fu) | (((qhv[i] >> sh_a) & 0x03030303u) << 4));
      vb[i] = static_cast<int>(((qlv[i] >> 4) & 0x0F0F0F0Fu) | (((qhv[i] >> sh_b) & 0x03030303u) << 4));
    }
#pragma unroll
    for (int c = 0; c < MC; ++c) {
      int dA = dot4(va[0], xa[c].x, -suma[c]);
      dA = dot4(va[1], xa[c].y, dA);
      dA = dot4(va[2], xa[c].z, dA);
      dA = dot4(va[3], xa[c].w, dA);
      int dB = dot4(vb[0], xb[c].x, -sumb[c]);
      dB = dot4(vb[1], xb[c].y, dB);
      dB = dot4(vb[2], xb[c].z, dB);
      dB = dot4(vb[3], xb[c].w, dB);
      acc[r][c] += dsa * da[c] * static_cast<float>(dA) + dsb * db[c] * static_cast<float>(dB);
    }
  }
}

// ---------------------------------------------------------------------------
// Q6_K, wide slices (MC <= 2): slice w (0..3) of super-block b is half
// g = w >> 1 (values 128g..128g+127) and sub-range h = w & 1: qh bytes
// 32g + 16h.. (16 bytes, each holding the top bits of 4 values) and the ql
// bytes 64g + 16h.. and 64g + 32 + 16h.. they pair with, i.e. values
// 128g + 32k + 16h + i for k = 0..3, i = 0..15 (scale 8g + 2k + h, Q8_1
// block 8b + 4g + k).  One lane per 64 weights; qh is read once.
// ---------------------------------------------------------------------------
// The weight bytes of wide Q6_K slice s of R rows, loaded before their use.
template <int R>
struct Q6Wide {
  u32x4 ql0[R], ql1[R], qh[R];
  u32x2 scw[R];
  uint16_t dbits[R];
};

// RS: the row-split Q6_K_R layout of a row of K values (ifx_common.h).
template <int R, bool RS = false>
__device__ __forceinline__ void q6k_wide_load(Q6Wide<R> &wt, const rsrc_t Wr,
                                              const uint32_t (&voff)[R], const uint32_t (&soff)[R],
                                              int s, int K = 0) {
  const int b = s >> 2, g = (s >> 1) & 1, h = s & 1;
  if constexpr (RS) {
    const uint32_t qh0 = K >> 1, sc0 = qh0 + (K >> 2), d0 = sc0 + (K >> 4);
#pragma unroll
    for (int r = 0; r < R; ++r) {
      wt.ql0[r] = wload<u32x4>(Wr, voff[r] + b * 128 + g * 64 + 16 * h, soff[r]);
      wt.ql1[r] = wload<u32x4>(Wr, voff[r] + b * 128 + g * 64 + 32 + 16 * h, soff[r]);
      wt.qh[r] = wload<u32x4>(Wr, voff[r] + qh0 + b * 64 + g * 32 + 16 * h, soff[r]);
      wt.scw[r] = wload<u32x2>(Wr, voff[r] + sc0 + b * 16 + g * 8, soff[r]);
      wt.dbits[r] = wload<uint16_t>(Wr, voff[r] + d0 + b * 2, soff[r]);
    }
    return;
  }
  const uint32_t wo = b * kQ6KBytes;
#pragma unroll
  for (int r = 0; r < R; ++r) {
    wt.ql0[r] = wload<u32x4>(Wr, voff[r] + wo + g * 64 + 16 * h, soff[r]);
    wt.ql1[r] = wload<u32x4>(Wr, voff[r] + wo + g * 64 + 32 + 16 * h, soff[r]);
    wt.qh[r] = wload<u32x4>(Wr, voff[r] + wo + 128 + g * 32 + 16 * h, soff[r]);
    wt.scw[r] = wload<u32x2>(Wr, voff[r] + wo + 192 + g * 8, soff[r]);
    wt.dbits[r] = wload<uint16_t>(Wr, voff[r] + wo + 208, soff[r]);
  }
}

// The activation words of wide Q6_K slice s (the 16 codes of this lane's
// half of Q8_1 blocks 8b + 4g + k, k = 0..3, and their d), as loaded.
template <int MC>
struct Q6WideAct {
  i32x4 x[4][MC];
  uint16_t dbits[4][MC];
};

template <int MC, typename AS>
__device__ __forceinline__ void q6k_wide_act(Q6WideAct<MC> &a, const AS &as, int mvalid, int s) {
  const int b = s >> 2, g = (s >> 1) & 1, h = s & 1;
#pragma unroll
  for (int c = 0; c < MC; ++c) {
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      if (c == 0 || c < mvalid) {  // mvalid >= 1
        const uint32_t ao = (b * 8 + g * 4 + k) * kQ8_1Bytes;
        a.x[k][c] = as.template get<i32x4>(ao + 4 + 16 * h, c);
        a.dbits[k][c] = as.template get<uint16_t>(ao, c);
      } else {
        a.x[k][c] = i32x4{0, 0, 0, 0};
        a.dbits[k][c] = 0;  // fp16 zero
      }
    }
  }
}

template <int MC, int R>
__device__ __forceinline__ void q6k_wide_math(const Q6Wide<R> &wt, const Q6WideAct<MC> &a, int s,
                                              float (&acc)[R][MC]) {
  const int h = s & 1;
  float da[4][MC];
  int sum32[4][MC];  // 32 * sum of the 16 activation codes (the -32 offset)
#pragma unroll
  for (int c = 0; c < MC; ++c) {
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      da[k][c] = h2f(a.dbits[k][c]);
      int sm = dot4(0x01010101, a.x[k][c].x, 0);
      sm = dot4(0x01010101, a.x[k][c].y, sm);
      sm = dot4(0x01010101, a.x[k][c].z, sm);
      sm = dot4(0x01010101, a.x[k][c].w, sm);
      sum32[k][c] = 32 * sm;
    }
  }
  const int scs = 8 * h;  // scale byte h (k = 0, 2) or h + 2 (k = 1, 3) of its dword
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const float d = h2f(wt.dbits[r]);
    // scales[8g + 2k + h]: dword 0 holds k = 0 (byte h) and k = 1 (byte h + 2),
    // dword 1 holds k = 2 and k = 3
    float dsk[4];
    dsk[0] = d * static_cast<float>(static_cast<int8_t>((wt.scw[r].x >> scs) & 0xFFu));
    dsk[1] = d * static_cast<float>(static_cast<int8_t>((wt.scw[r].x >> (scs + 16)) & 0xFFu));
    dsk[2] = d * static_cast<float>(static_cast<int8_t>((wt.scw[r].y >> scs) & 0xFFu));
    dsk[3] = d * static_cast<float>(static_cast<int8_t>((wt.scw[r].y >> (scs + 16)) & 0xFFu));
    const uint32_t l0[4] = {wt.ql0[r].x, wt.ql0[r].y, wt.ql0[r].z, wt.ql0[r].w};
    const uint32_t l1[4] = {wt.ql1[r].x, wt.ql1[r].y, wt.ql1[r].z, wt.ql1[r].w};
    const uint32_t hv[4] = {wt.qh[r].x, wt.qh[r].y, wt.qh[r].z, wt.qh[r].w};
    int v[4][4];  // 6-bit codes of value group k, dword i
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[0][i] = static_cast<int>((l0[i] & 0x0F0F0F0Fu) | ((hv[i] << 4) & 0x30303030u));
      v[1][i] = static_cast<int>((l1[i] & 0x0F0F0F0Fu) | ((hv[i] << 2) & 0x30303030u));
      v[2][i] = static_cast<int>(((l0[i] >> 4) & 0x0F0F0F0Fu) | (hv[i] & 0x30303030u));
      v[3][i] = static_cast<int>(((l1[i] >> 4) & 0x0F0F0F0Fu) | ((hv[i] >> 2) & 0x30303030u));
    }
#pragma unroll
    for (int c = 0; c < MC; ++c) {
      float sum = 0.0f;
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        int dt = dot4(v[k][0], a.x[k][c].x, -sum32[k][c]);
        dt = dot4(v[k][1], a.x[k][c].y, dt);
        dt = dot4(v[k][2], a.x[k][c].z, dt);
        dt = dot4(v[k][3], a.x[k][c].w, dt);
        sum += dsk[k] * da[k][c] * static_cast<float>(dt);
      }
      acc[r][c] += sum;
    }
  }
}

template <int MC, int R, bool RS = false>
__device__ __forceinline__ void q6k_wide(const rsrc_t Wr, rsrc_t Ar, const uint32_t (&voff)[R],
                                         const uint32_t (&soff)[R], uint32_t a_row, int mvalid,
                                         int s, float (&acc)[R][MC], int K = 0) {
  // weight and activation loads issued together, before any wait: left to
  // itself the scheduler issued the activation loads only after the weights
  // had landed, a second dependent round trip per slice (3B down at M = 1:
  // 7.24 -> 6.89 us raw, 6.80 -> 6.75 row-split)
  Q6Wide<R> wt;
  q6k_wide_load<R, RS>(wt, Wr, voff, soff, s, K);
  Q6WideAct<MC> a;
  q6k_wide_act<MC>(a, AGlobal{Ar, a_row}, mvalid, s);
  __builtin_amdgcn_sched_barrier(0);
  q6k_wide_math<MC, R>(wt, a, s, acc);
}

}  // namespace ifx
