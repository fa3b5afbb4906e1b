// gemv.hip -- weight-streaming GEMV for the decode batch (M <= 8) on gfx950:
// y[m][n] = sum_k W[n][k] * a[m][k] with W raw GGUF Q4_K / Q6_K / Q8_0 blocks
// and a Q8_1 blocks of 32.
//
// Replaces the reference's MMVQ kernels
// (runtime/backends/cuda/native/kernels/mmvq.cuh:49-158 Q4_K, 407-843 Q6_K,
// 843-1019 Q8_0, with the accumulate/bias epilogues at 163-401) and keeps
// their arithmetic: an integer dot over each 32-value (Q4_K, Q8_0) or
// 16-value (Q6_K) run, then fp32 scaling; the Q4_K min term uses the Q8_1
// s = d*sum(q) field (mmvq.cuh:121-125).
//
// Work mapping (wave64, memory bound):
//  * A "slice" is the run of weights one lane owns.  At M <= 2 (Q6_K: M = 1)
//    Q4_K and Q6_K use wide 64-value slices (32 bytes of Q4_K qs = one
//    sub-block pair; 32 bytes of Q6_K ql + the 16 bytes of qh they share):
//    the kernel is VALU co-limited there, and the per-slice costs (header
//    broadcast, scale/min decode, activation scales) are paid once per 64
//    weights.  Otherwise a slice is 32 weights: 16 bytes of Q4_K qs (two
//    half sub-blocks), 16 bytes of Q6_K ql plus the matching 16 bytes of
//    qh, or one whole Q8_0 block.
//  * Half-wave mode (wide slices, K <= 2048, i.e. at most 32 slices a row):
//    lanes 0-31 and 32-63 own different rows, so no lane idles.
//  * A row group of R consecutive rows is owned by G waves (G = 1..4 by K,
//    so that 64*G lanes roughly cover K/32 slices); lane t of the group
//    takes slices t, t + 64G, ...  For each slice a lane loads the
//    activation codes and scales of all MC batch columns once and reuses
//    them across the R rows, then issues the weight loads of all R rows
//    before using any, so a lane keeps R*32 bytes (Q4_K) in flight.
//  * Rows past N are clamped (loaded but never stored), so no branch
//    separates a lane's loads.
//  * Partial sums acc[R*MC] are combined across the 64 lanes of a wave with
//    DPP adds (no LDS traffic; lane 63 ends with the totals), then across
//    the G waves of the group through LDS.
//  * Q4_K header (16 bytes per super-block): with 32-value slices it is
//    loaded by one of the eight lanes that share it and broadcast with DPP;
//    with wide slices each of the four lanes loads it (measured faster).
#include "ifx_slices.h"

#include <stdlib.h>

namespace ifx {

// ---------------------------------------------------------------------------
// Q8_0: slice s is block s of the row (34 bytes: fp16 d, 32 int8 codes).
// ---------------------------------------------------------------------------
// K8 = true: Q8_K (mmvq.cuh:1019-1070): slice s is codes 32(s&7).. of
// super-block s>>3 (292 bytes: fp32 d, i8 qs[256], i16 bsums[16]); the
// fp32 d is shared by the eight slices of a super-block.
// RS = true: the row-split Q8_0_R layout (ifx_common.h): codes at 32 s,
// d at K + 2 s.
template <int MC, int R, bool K8 = false, bool RS = false>
__device__ __forceinline__ void q8_0_slice(const rsrc_t (&Wr)[R], rsrc_t Ar, const uint32_t (&rows)[R],
                                           uint32_t a_row, int mvalid, int s, float (&acc)[R][MC],
                                           int K = 0) {
  i32x4 w0[R], w1[R];
  uint32_t dbits[R];
  const uint32_t wo = RS ? K + 2 * s : K8 ? (s >> 3) * kQ8KBytes : s * kQ8_0Bytes;
  const uint32_t qo = RS ? 32 * s : K8 ? wo + 4 + 32 * (s & 7) : wo + 2;
#pragma unroll
  for (int r = 0; r < R; ++r) {
    if constexpr (K8) dbits[r] = wload<uint32_t>(Wr[r], wo, rows[r]);
    else dbits[r] = wload<uint16_t>(Wr[r], wo, rows[r]);
    w0[r] = wload<i32x4>(Wr[r], qo, rows[r]);
    w1[r] = wload<i32x4>(Wr[r], qo + 16, rows[r]);
  }
  i32x4 x0[MC], x1[MC];
  float da[MC];
#pragma unroll
  for (int c = 0; c < MC; ++c) {
    if (c == 0 || c < mvalid) {  // mvalid >= 1
      const uint32_t ao = s * kQ8_1Bytes;
      x0[c] = bload<i32x4>(Ar, ao + 4, c * a_row);
      x1[c] = bload<i32x4>(Ar, ao + 20, c * a_row);
      da[c] = h2f(bload<uint16_t>(Ar, ao, c * a_row));
    } else {
      x0[c] = x1[c] = i32x4{0, 0, 0, 0};
      da[c] = 0.0f;
    }
  }
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const float d = K8 ? __builtin_bit_cast(float, dbits[r]) : h2f(dbits[r] & 0xFFFFu);
#pragma unroll
    for (int c = 0; c < MC; ++c) {
      int dt = dot4(w0[r].x, x0[c].x, 0);
      dt = dot4(w0[r].y, x0[c].y, dt);
      dt = dot4(w0[r].z, x0[c].z, dt);
      dt = dot4(w0[r].w, x0[c].w, dt);
      dt = dot4(w1[r].x, x1[c].x, dt);
      dt = dot4(w1[r].y, x1[c].y, dt);
      dt = dot4(w1[r].z, x1[c].z, dt);
      dt = dot4(w1[r].w, x1[c].w, dt);
      acc[r][c] += d * da[c] * static_cast<float>(dt);
    }
  }
}

// ---------------------------------------------------------------------------
// Kernel.  blockDim = 64 * G * P: P row groups of G waves.  blockIdx.y
// selects the group of MC batch columns.  blockIdx.x walks the row groups of
// up to kMaxSeg projections that share the activations A (the reference's
// grouped pair/triple launches, mmvq.cuh:1197-1448): workgroups
// [seg[i].blk_begin, seg[i + 1].blk_begin) belong to projection i.
// ---------------------------------------------------------------------------
constexpr int kMaxSeg = 3;

struct GemvSeg {
  const uint8_t *W;
  void *Y;
  const void *bias;
  int N;
  int blk_begin;
};

struct GemvArgs {
  GemvSeg seg[kMaxSeg];
  int nseg;
  const uint8_t *A;
  int M, K, mode;
  // fused RMSNorm producer (NORM != 0): residual x [M][K] (fp32 or fp16)
  // and norm weight [K] fp16; A is not read
  const void *x;
  const uint16_t *norm_w;
  float eps;
};

// The segment of workgroup bx.  All segments' fields are read at once and
// selected: an indexed read (args.seg[si]) waits for the index, one more
// dependent scalar-memory round trip before the first weight load can
// issue, in every wave of the launch.
__device__ __forceinline__ GemvSeg pick_seg(const GemvArgs &a, int bx) {
  const GemvSeg s0 = a.seg[0], s1 = a.seg[1], s2 = a.seg[2];
  const bool in2 = a.nseg > 2 && bx >= s2.blk_begin;
  const bool in1 = !in2 && a.nseg > 1 && bx >= s1.blk_begin;
  GemvSeg g;
  g.W = in2 ? s2.W : in1 ? s1.W : s0.W;
  g.Y = in2 ? s2.Y : in1 ? s1.Y : s0.Y;
  g.bias = in2 ? s2.bias : in1 ? s1.bias : s0.bias;
  g.N = in2 ? s2.N : in1 ? s1.N : s0.N;
  g.blk_begin = in2 ? s2.blk_begin : in1 ? s1.blk_begin : s0.blk_begin;
  return g;
}

// Q4_K with MC <= 2 and Q6_K with MC = 1 use the wide (64-value) slices
// (Q6_K at MC = 2 is faster with 32-value slices: fewer registers).  H = 2 (half-wave
// mode, wide slices, K <= 2048 so that one row needs at most 32 lanes):
// lanes 0-31 and 32-63 own different sets of R rows.
template <int QT, int MC>
constexpr bool kWide = (QT == kTypeQ4_K && MC <= 2) ||
                       ((QT == kTypeQ6_K || QT == kTypeQ6_KR) && MC == 1);

// NORM = 1 / 2: the activations are produced in the kernel from an fp32 /
// fp16 residual (RMSNorm then Q8_1, the standalone producer's exact
// arithmetic) into LDS; NORM = 3 / 4: from fp32 / fp16 activations by the
// plain Q8_1 quantizer (the standalone quantizer's blocks, bit for bit).  For K <= 2048 the residual and norm-weight loads
// are issued first, then the first slice's weight loads, and the norm is
// computed while the weights stream in (a wave's loads complete in order);
// larger K runs the norm before the first weight load.  Wide Q4_K slices and
// 256-thread workgroups only.
template <int QT, int MC, int R, int G, int P, bool F16OUT, int H, int NORM = 0, bool EB = false>
__global__ __launch_bounds__(64 * G * P) void k_gemv(const GemvArgs args) {
  static_assert(H == 1 || (G == 1 && kWide<QT, MC>), "sub-wave rows: wide slices, one wave per row group");
  static_assert(NORM == 0 || (QT == kTypeQ4_K && kWide<QT, MC> && 64 * G * P == 256),
                "fused RMSNorm: wide Q4_K slices, 256 threads");
  constexpr int V = R * MC;  // partial sums per lane; a power of two <= 64
  constexpr int LPR = 64 / H;                       // lanes per row set
  constexpr int SV = kWide<QT, MC> ? 64 : 32;       // values per slice
  __shared__ float red[(G > 1) ? P * G * V : 1];
  [[maybe_unused]] constexpr int kStampBase = NORM == 1 ? 0 : NORM == 3 ? 1 : 3;
  IFX_STAMP(0);
  const int bx = blockIdx.x;
  const GemvSeg sg = pick_seg(args, bx);
  // the activation pointer is needed by every lane; using it here keeps its
  // kernel-argument load in the first batch rather than behind a branch
  asm volatile("" ::"s"(args.A));
  const uint8_t *__restrict__ W = sg.W;
  const int N = sg.N, M = args.M, K = args.K, mode = args.mode;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform
  const int gw = wave % G;   // wave within its row group
  const int grp = wave / G;  // row group within the workgroup
  const int half = (H >= 2) ? (lane / (64 / H)) : 0;  // row set of this lane
  const int lt = lane & (LPR - 1);  // lane within its row set
  const int row0 = (((bx - sg.blk_begin) * P + grp) * H + half) * R;
  const int col0 = blockIdx.y * MC;
  const int mvalid = min(MC, M - col0);
  const uint32_t a_row = static_cast<uint32_t>(K >> 5) * kQ8_1Bytes;
  const uint32_t w_row = static_cast<uint32_t>(row_bytes(QT, K));
  // 32-bit ranges (the launcher checks the tensors are below 4 GiB)
  const rsrc_t Wr = make_rsrc(W, w_row * static_cast<uint32_t>(N));
  const rsrc_t Ar = make_rsrc(args.A + static_cast<int64_t>(col0) * a_row, a_row * mvalid);

  uint32_t rows[R];  // byte offset of each row (rows past N repeat row N-1)
  rsrc_t Wrs[R];     // the tensor each row is read from
#pragma unroll
  for (int r = 0; r < R; ++r) {
    rows[r] = static_cast<uint32_t>(min(row0 + r, N - 1)) * w_row;
    Wrs[r] = Wr;
  }
  // wide slices: row offsets go in voffset when they differ per lane (H = 2),
  // in soffset when they are wave-uniform
  uint32_t voff[R], soff[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    voff[r] = (H >= 2) ? rows[r] : 0u;
    soff[r] = (H >= 2) ? 0u : rows[r];
  }

  float acc[R][MC];
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int c = 0; c < MC; ++c) acc[r][c] = 0.0f;

  // EB (accumulate and bias launches): the term each output this lane may
  // store adds, loaded ahead of the weights and without a branch, so that
  // the epilogue waits on no dependent load (nothing else writes these
  // outputs during the launch: the value is the one a load at the end would
  // see; 3B down / O at M = 1: 7.14 -> 6.81 / 3.39 -> 3.22 us).  Indices are
  // clamped where the value goes unused.  Up to 8 values a lane; more keep
  // the load at the end.
  constexpr bool kEarlyBase = EB && V <= 8;
  float base[kEarlyBase ? V : 1];
  if constexpr (kEarlyBase) {
    const bool bias_mode = mode == kOutBias;
#pragma unroll
    for (int idx = 0; idx < V; ++idx) {
      const int row = min(row0 + idx / MC, N - 1);
      const int64_t o = static_cast<int64_t>(col0 + min(idx % MC, mvalid - 1)) * N + row;
      const int64_t at = bias_mode ? row : o;  // no offset from a null bias
      if constexpr (F16OUT)
        base[idx] = h2f(static_cast<const uint16_t *>(bias_mode ? sg.bias : sg.Y)[at]);
      else
        base[idx] = static_cast<const float *>(bias_mode ? sg.bias : sg.Y)[at];
    }
  }

  const int nslice = K / SV;
  if constexpr (NORM != 0) {
    constexpr bool kXF16 = NORM == 2 || NORM == 4, kRms = NORM <= 2;
    extern __shared__ __attribute__((aligned(16))) uint8_t a_lds[];  // [MC] split rows
    const uint32_t a_str = split_row_bytes(K);
    __shared__ float npart[4 * MC];
    const int s0 = gw * LPR + lt;
    Q4Wide<R> wt;
    if (K <= 2048) {
      // activations (and norm weight) first, then the first slice's
      // weights: the producer's inputs arrive without waiting for the
      // weight stream
      f32x4 xr[MC][2];
      u32x2 wr[MC][2];
#pragma unroll
      for (int c = 0; c < MC; ++c)  // columns past M re-read the last one (unused)
        rmsnorm_row_load_nb<kXF16, 2, kRms>(args.x, static_cast<int64_t>(col0 + min(c, mvalid - 1)) * K,
                                            args.norm_w, K, threadIdx.x, xr[c], wr[c]);
      // keep the activation loads ahead of the weight loads in issue order
      __atomic_signal_fence(__ATOMIC_SEQ_CST);
      __builtin_amdgcn_sched_barrier(0);
      q4k_wide_load<R>(wt, Wr, voff, soff, min(s0, nslice - 1));  // unconditional: no wait on it
#pragma unroll
      for (int c = 0; c < MC; ++c)
        if (c < mvalid) {
          if constexpr (kRms)
            rmsnorm_row_finish<2, true>(xr[c], wr[c], a_lds + c * a_str, K, args.eps, npart + 4 * c,
                                  threadIdx.x);
          else
            quantize_row_finish<2, true>(xr[c], a_lds + c * a_str, K, threadIdx.x);
        }
    } else {
#pragma unroll
      for (int c = 0; c < MC; ++c)
        if (c < mvalid) {
          if constexpr (kRms)
            rmsnorm_quantize_row<kXF16, true>(args.x, static_cast<int64_t>(col0 + c) * K, args.norm_w,
                                        a_lds + c * a_str, K, args.eps, npart + 4 * c,
                                        threadIdx.x);
          else
            quantize_row<kXF16, true>(args.x, static_cast<int64_t>(col0 + c) * K, a_lds + c * a_str, K,
                                threadIdx.x);
        }
      if (s0 < nslice) q4k_wide_load<R>(wt, Wr, voff, soff, s0);
    }
    __syncthreads();
    IFX_STAMP(1);
    const ALdsS as{a_lds, a_str, static_cast<uint32_t>(K / 64 * 80)};
    for (int s = s0; s < nslice; s += LPR * G) {
      if (s != s0) q4k_wide_load<R>(wt, Wr, voff, soff, s);
      q4k_wide_compute<MC, R>(wt, as, mvalid, s, acc);
    }
  } else
  for (int s = gw * LPR + lt; s < nslice; s += LPR * G) {
    if constexpr (kWide<QT, MC> && QT == kTypeQ4_K)
      q4k_wide<MC, R>(Wr, Ar, voff, soff, a_row, mvalid, s, acc);
    else if constexpr (kWide<QT, MC>)
      q6k_wide<MC, R, QT == kTypeQ6_KR>(Wr, Ar, voff, soff, a_row, mvalid, s, acc, K);
    else if constexpr (QT == kTypeQ4_K)
      q4k_slice<MC, R>(Wrs, Ar, rows, a_row, mvalid, s, acc);
    else if constexpr (QT == kTypeQ5_K)
      q4k_slice<MC, R, true>(Wrs, Ar, rows, a_row, mvalid, s, acc);
    else if constexpr (QT == kTypeQ6_K)
      q6k_slice<MC, R>(Wrs, Ar, rows, a_row, mvalid, s, acc);
    else if constexpr (QT == kTypeQ6_KR)
      q6k_slice<MC, R, true>(Wrs, Ar, rows, a_row, mvalid, s, acc, K);
    else if constexpr (QT == kTypeQ8_K)
      q8_0_slice<MC, R, true>(Wrs, Ar, rows, a_row, mvalid, s, acc);
    else if constexpr (QT == kTypeQ8_0R)
      q8_0_slice<MC, R, false, true>(Wrs, Ar, rows, a_row, mvalid, s, acc, K);
    else
      q8_0_slice<MC, R>(Wrs, Ar, rows, a_row, mvalid, s, acc);
  }

  IFX_STAMP(2);
  // Sum each partial over the wave (DPP adds, no LDS); lane 63 ends with
  // all V totals, then across the G waves of the row group through LDS.
  float v[V];
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int c = 0; c < MC; ++c)
      v[r * MC + c] = (H == 4)   ? quarterwave_sum(acc[r][c])
                      : (H == 2) ? halfwave_sum_to31(acc[r][c])
                                 : wave_sum_to63(acc[r][c]);
  if constexpr (G > 1) {
    if (lane == 63) {
#pragma unroll
      for (int i = 0; i < V; ++i) red[(grp * G + gw) * V + i] = v[i];
    }
    __syncthreads();
    if (gw != 0 || lane != 63) return;
#pragma unroll
    for (int i = 0; i < V; ++i) {
      float t = 0.0f;
#pragma unroll
      for (int w = 0; w < G; ++w) t += red[(grp * G + w) * V + i];
      v[i] = t;
    }
  } else {
    if ((lane & (LPR - 1)) != LPR - 1) return;
  }
#pragma unroll
  for (int idx = 0; idx < V; ++idx) {
    float y = v[idx];
    const int r = idx / MC, c = idx % MC;
    const int row = row0 + r;
    if (row >= N || c >= mvalid) continue;
    const int64_t o_idx = static_cast<int64_t>(col0 + c) * N + row;
    if constexpr (F16OUT) {
      uint16_t *Yh = static_cast<uint16_t *>(sg.Y);
      if constexpr (kEarlyBase) {
        if (mode == kOutAccum || mode == kOutBias) y += base[idx];
      } else if (mode == kOutAccum) {
        y += h2f(Yh[o_idx]);
      } else if (mode == kOutBias) {
        y += h2f(static_cast<const uint16_t *>(sg.bias)[row]);
      }
      Yh[o_idx] = static_cast<uint16_t>(f2h_bits(y));
    } else {
      float *Yf = static_cast<float *>(sg.Y);
      if constexpr (kEarlyBase) {
        if (mode == kOutAccum || mode == kOutBias) y += base[idx];
      } else if (mode == kOutAccum) {
        y += Yf[o_idx];
      } else if (mode == kOutBias) {
        y += static_cast<const float *>(sg.bias)[row];
      }
      Yf[o_idx] = y;
    }
  }
  IFX_STAMP(3);
}

template <int QT, int MC, int R, int G, int H = 1>
static void launch_t(GemvArgs args, bool f16, hipStream_t s) {
  constexpr int P = (G >= 3) ? 1 : 4 / G;
  int blocks = 0;
  for (int i = 0; i < args.nseg; ++i) {
    args.seg[i].blk_begin = blocks;
    const int groups = (args.seg[i].N + H * R - 1) / (H * R);
    blocks += (groups + P - 1) / P;
  }
  const dim3 grid(blocks, (args.M + MC - 1) / MC);
  const dim3 block(64 * G * P);
  const bool eb = args.mode != kOutStore;
  if (f16 && eb)
    IFX_LAUNCH(k_gemv, (QT, MC, R, G, P, true, H, 0, true), grid, block, 0, s, args);
  else if (f16)
    IFX_LAUNCH(k_gemv, (QT, MC, R, G, P, true, H), grid, block, 0, s, args);
  else if (eb)
    IFX_LAUNCH(k_gemv, (QT, MC, R, G, P, false, H, 0, true), grid, block, 0, s, args);
  else
    IFX_LAUNCH(k_gemv, (QT, MC, R, G, P, false, H), grid, block, 0, s, args);
}

// Rows per wave section: IFX_GEMV_H in {1, 2, 4} forces full-, half- or
// quarter-wave rows for the wide slices (tuning; read once).
static int sub_rows_env() {
  static const int env = [] {
    const char *e = ifx::tuning_env("IFX_GEMV_H");
    const int v = e ? atoi(e) : 0;
    return (v == 1 || v == 2 || v == 4) ? v : 0;
  }();
  return env;
}

// Quarter-wave rows (16 lanes) when they leave no lane idle and the full-wave
// launch would: e.g. K = 5120 has 80 wide slices, 5 per lane on 16 lanes
// against 80 of 128 lanes busy on two waves.  Measured on the 14B shapes
// (K = 5120): M = 1 QKV 6.7 -> 5.7 us, gate+up 19.3 -> 18.4 us; at M = 2
// only launches of >= 8192 rows gain (gate+up 22.9 -> 20.9 us; QKV and O
// lose), hence the launcher's rule.
static bool quarter_rows(int nslice) {
  return nslice % 16 == 0 && nslice % 64 != 0 && nslice <= 16 * 8;
}

// Lanes per row of a wide-slice launch: 64 / the result (1: full-wave rows,
// possibly several waves per row).  The fused-RMSNorm launch uses the same
// rule, so its row sums are formed in the same order as the plain GEMV's.
template <int MC>
static int wide_sub_rows(const GemvArgs &args, int nslice) {
  if (sub_rows_env()) return sub_rows_env();
  int n_total = 0;
  for (int i = 0; i < args.nseg; ++i) n_total += args.seg[i].N;
  if (nslice > 32 && quarter_rows(nslice) && (MC == 1 || n_total >= 8192)) return 4;
  return nslice <= 32 ? 2 : 1;
}

template <int QT, int MC, int R>
static void launch_g(const GemvArgs &args, bool f16, hipStream_t s) {
  // waves per row group: enough lanes to cover the slices, at most 4; a
  // row of at most 32 wide slices takes half a wave
  const int nslice = args.K / (kWide<QT, MC> ? 64 : 32);
  const int g = (nslice + 63) / 64;
  if constexpr (kWide<QT, MC>) {
    const int h = wide_sub_rows<MC>(args, nslice);
    if (h == 4) {
      launch_t<QT, MC, R, 1, 4>(args, f16, s);
      return;
    }
    if (h == 2) {
      launch_t<QT, MC, R, 1, 2>(args, f16, s);
      return;
    }
  }
  if (g <= 1) launch_t<QT, MC, R, 1>(args, f16, s);
  else if (g == 2) launch_t<QT, MC, R, 2>(args, f16, s);
  else if (g == 3) launch_t<QT, MC, R, 3>(args, f16, s);
  else launch_t<QT, MC, R, 4>(args, f16, s);
}

// Rows per wave (R; a half-wave launch covers 2R): enough waves to keep
// ~4 per SIMD in flight on small N, more rows per wave (more bytes in
// flight per lane) on large N.  Measured on MI355X with cold weights (each
// launch reads a copy not in the 256 MB Infinity Cache), M = 1 / 2:
//  * 32-value slices: N = 2048 -> 1 (2 when K >= 8192), N = 11008/13824
//    -> 2, N = 151936 -> 4;
//  * wide Q4_K slices: half-wave R = 1 for N < 8192, else 2 (4 rows a
//    wave); full-wave R = M for N < 8192, else 2M;
//  * wide Q6_K slices: R = 2 below N = 4096, else 4; row-split Q8_0 at
//    M = 1, N >= 65536: 1.
// IFX_GEMV_ROWS in {1, 2, 4, 8} overrides it (tuning; read once).
static int rows_env() {
  static const int env = [] {
    const char *e = ifx::tuning_env("IFX_GEMV_ROWS");
    const int v = e ? atoi(e) : 0;
    return (v == 1 || v == 2 || v == 4 || v == 8) ? v : 0;
  }();
  return env;
}

template <int QT, int MC>
static int rows_per_wave(int N, int K) {
  if (rows_env()) return rows_env();
  // wide Q6_K (activation loads issued with the weights): 4 rows a wave
  // from N = 4096 (LM head 151936 x 2048: 56 -> 50 us raw, 46 -> 44.4
  // row-split; 14B down 5120 x 13824: 16.4 -> 15.6 us), 2 below (3B down
  // 2048 x 11008: 6.6 against 6.9 at 4)
  if constexpr (kWide<QT, MC> && (QT == kTypeQ6_K || QT == kTypeQ6_KR)) return N >= 4096 ? 4 : 2;
  // row-split Q8_0, one column, LM-head sized launches: the aligned rows
  // stream best one per wave (151936 x 2048: 51.5 against 54.2 us at 4)
  if constexpr (QT == kTypeQ8_0R && MC == 1)
    if (N >= 65536) return 1;
  if constexpr (kWide<QT, MC>) {
    const bool half = K / 64 <= 32;  // half-wave launch: a wave covers 2R rows
    if (N < 8192) return half ? 1 : MC;
    return half ? 2 : 2 * MC;
  }
  return N < 8192 ? (K >= 8192 ? 2 : 1) : N < 65536 ? 2 : 4;
}

template <int QT, int MC>
static void launch_r(const GemvArgs &args, bool f16, hipStream_t s) {
  int n_total = 0;
  for (int i = 0; i < args.nseg; ++i) n_total += args.seg[i].N;
  switch (rows_per_wave<QT, MC>(n_total, args.K)) {
  case 1: launch_g<QT, MC, 1>(args, f16, s); break;
  case 2: launch_g<QT, MC, 2>(args, f16, s); break;
  case 8: launch_g<QT, MC, 8>(args, f16, s); break;
  default: launch_g<QT, MC, 4>(args, f16, s); break;
  }
}

// The GEMV with the fused RMSNorm producer (Q4_K wide slices, M <= 2):
// the row geometry of launch_g, 256-thread workgroups (3 waves per row
// group become 4), the Q8_1 activations of the MC columns in dynamic LDS.
template <int MC, int R, int G, int H, int NORM>
static void launch_norm_t(GemvArgs args, bool f16, hipStream_t s) {
  constexpr int P = 4 / G;
  int blocks = 0;
  for (int i = 0; i < args.nseg; ++i) {
    args.seg[i].blk_begin = blocks;
    const int groups = (args.seg[i].N + H * R - 1) / (H * R);
    blocks += (groups + P - 1) / P;
  }
  const dim3 grid(blocks, (args.M + MC - 1) / MC);
  const size_t shm = static_cast<size_t>(MC) * split_row_bytes(args.K);
  const bool eb = args.mode != kOutStore;
  if (f16 && eb)
    IFX_LAUNCH(k_gemv, (kTypeQ4_K, MC, R, G, P, true, H, NORM, true), grid, dim3(256), shm, s,
                       args);
  else if (f16)
    IFX_LAUNCH(k_gemv, (kTypeQ4_K, MC, R, G, P, true, H, NORM), grid, dim3(256), shm, s,
                       args);
  else if (eb)
    IFX_LAUNCH(k_gemv, (kTypeQ4_K, MC, R, G, P, false, H, NORM, true), grid, dim3(256), shm, s,
                       args);
  else
    IFX_LAUNCH(k_gemv, (kTypeQ4_K, MC, R, G, P, false, H, NORM), grid, dim3(256), shm, s,
                       args);
}

template <int MC, int R, int NORM>
static void launch_norm_g(const GemvArgs &args, bool f16, hipStream_t s) {
  const int nslice = args.K / 64;
  const int g = (nslice + 63) / 64;
  const int h = wide_sub_rows<MC>(args, nslice);
  if (h == 4) launch_norm_t<MC, R, 1, 4, NORM>(args, f16, s);
  else if (h == 2) launch_norm_t<MC, R, 1, 2, NORM>(args, f16, s);
  else if (g <= 1) launch_norm_t<MC, R, 1, 1, NORM>(args, f16, s);
  else if (g == 2) launch_norm_t<MC, R, 2, 1, NORM>(args, f16, s);
  else launch_norm_t<MC, R, 4, 1, NORM>(args, f16, s);
}

// Rows per wave as the plain GEMV, except that a single column with the
// RMSNorm prologue takes at least 2 (half-wave rows: 4 rows a wave), so
// fewer workgroups repeat the norm: 3B QKV (2560 rows) 3.84 -> 3.35 us,
// while the quantize-only prologue (O, 2048 rows) stays faster at 1 (3.25
// against 3.43 us).  The row sums do not depend on it.
template <int MC, int NORM>
static void launch_norm_r(const GemvArgs &args, bool f16, hipStream_t s) {
  int n_total = 0;
  for (int i = 0; i < args.nseg; ++i) n_total += args.seg[i].N;
  int r = rows_per_wave<kTypeQ4_K, MC>(n_total, args.K);
  if (MC == 1 && NORM <= 2 && r == 1 && !rows_env()) r = 2;
  switch (r) {
  case 1: launch_norm_g<MC, 1, NORM>(args, f16, s); break;
  case 2: launch_norm_g<MC, 2, NORM>(args, f16, s); break;
  default: launch_norm_g<MC, 4, NORM>(args, f16, s); break;
  }
}

template <int QT>
static void launch_type(const GemvArgs &args, bool f16, hipStream_t s) {
  if (args.M == 1) launch_r<QT, 1>(args, f16, s);
  else if (args.M == 2) launch_r<QT, 2>(args, f16, s);
  else if (args.M <= 4) launch_g<QT, 4, 4>(args, f16, s);
  else launch_g<QT, 8, 4>(args, f16, s);
}

// The row-split layouts run at M <= 2 only (checked by the caller).
template <int QT>
static void launch_m12(const GemvArgs &args, bool f16, hipStream_t s) {
  if (args.M == 1) launch_r<QT, 1>(args, f16, s);
  else launch_r<QT, 2>(args, f16, s);
}

static hipError_t launch_args(int qtype, const GemvArgs &args, bool f16, hipStream_t stream) {
  switch (qtype) {
  case kTypeQ4_K: launch_type<kTypeQ4_K>(args, f16, stream); break;
  case kTypeQ6_K: launch_type<kTypeQ6_K>(args, f16, stream); break;
  case kTypeQ8_0: launch_type<kTypeQ8_0>(args, f16, stream); break;
  case kTypeQ5_K: launch_type<kTypeQ5_K>(args, f16, stream); break;
  case kTypeQ8_K: launch_type<kTypeQ8_K>(args, f16, stream); break;
  case kTypeQ8_0R: launch_m12<kTypeQ8_0R>(args, f16, stream); break;
  case kTypeQ6_KR: launch_m12<kTypeQ6_KR>(args, f16, stream); break;
  default: return hipErrorInvalidValue;
  }
  return last_error();
}

// ---------------------------------------------------------------------------
// Fused gate/up GEMV with SiLU(gate) * up and a Q8_1 epilogue (replaces the
// reference's FusedGateUpSiluGemvQ8_1[WithEpilogue], mmvq.cuh:1686-2030):
// h[m][o] = silu(gate[o] . a[m]) * (up[o] . a[m]), written as fp32/fp16
// and/or as Q8_1 blocks of 32 consecutive outputs, ready for the down
// projection.  A workgroup of 16 waves owns 32 consecutive outputs (one Q8_1
// block per batch column): wave w computes outputs 2w and 2w+1 from the
// rows gate[o], gate[o+1], up[o], up[o+1] (one lane per 32-value slice),
// puts its h values in LDS, and after one barrier 8 lanes per batch column
// quantize the block with the standard quantizer.  (The reference's
// epilogue writes a per-element scale; this one is the full Q8_1 block.)
// ---------------------------------------------------------------------------
template <int QT, int MC, bool F16H>
__global__ __launch_bounds__(1024) void k_gemv_swiglu(const uint8_t *__restrict__ Wg,
                                                      const uint8_t *__restrict__ Wu,
                                                      const uint8_t *__restrict__ A,
                                                      void *__restrict__ H,
                                                      uint8_t *__restrict__ Q, int M, int N,
                                                      int K) {
  constexpr int R = 4, V = R * MC;
  __shared__ float hb[MC][32];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int o0 = blockIdx.x * 32 + 2 * wave;  // this wave's two outputs
  const int col0 = blockIdx.y * MC;
  const int mvalid = min(MC, M - col0);
  const int nslice = K >> 5;
  const uint32_t a_row = static_cast<uint32_t>(nslice) * kQ8_1Bytes;
  const uint32_t w_row = static_cast<uint32_t>(row_bytes(QT, K));
  const rsrc_t Wgr = make_rsrc(Wg, w_row * static_cast<uint32_t>(N));
  const rsrc_t Wur = make_rsrc(Wu, w_row * static_cast<uint32_t>(N));
  const rsrc_t Ar = make_rsrc(A + static_cast<int64_t>(col0) * a_row, a_row * mvalid);
  const uint32_t r0 = static_cast<uint32_t>(o0) * w_row;
  const uint32_t rows[R] = {r0, r0 + w_row, r0, r0 + w_row};
  const rsrc_t Wrs[R] = {Wgr, Wgr, Wur, Wur};

  float acc[R][MC];
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int c = 0; c < MC; ++c) acc[r][c] = 0.0f;
  for (int s = lane; s < nslice; s += 64) {
    if constexpr (QT == kTypeQ4_K)
      q4k_slice<MC, R>(Wrs, Ar, rows, a_row, mvalid, s, acc);
    else if constexpr (QT == kTypeQ5_K)
      q4k_slice<MC, R, true>(Wrs, Ar, rows, a_row, mvalid, s, acc);
    else if constexpr (QT == kTypeQ6_K)
      q6k_slice<MC, R>(Wrs, Ar, rows, a_row, mvalid, s, acc);
    else if constexpr (QT == kTypeQ6_KR)
      q6k_slice<MC, R, true>(Wrs, Ar, rows, a_row, mvalid, s, acc, K);
    else if constexpr (QT == kTypeQ8_K)
      q8_0_slice<MC, R, true>(Wrs, Ar, rows, a_row, mvalid, s, acc);
    else if constexpr (QT == kTypeQ8_0R)
      q8_0_slice<MC, R, false, true>(Wrs, Ar, rows, a_row, mvalid, s, acc, K);
    else
      q8_0_slice<MC, R>(Wrs, Ar, rows, a_row, mvalid, s, acc);
  }
  float v[V];
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int c = 0; c < MC; ++c) v[r * MC + c] = wave_sum_to63(acc[r][c]);
  if (lane == 63) {
#pragma unroll
    for (int c = 0; c < MC; ++c)
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const float gsum = v[t * MC + c], usum = v[(2 + t) * MC + c];
        const float h = materialize_f32(gsum / (1.0f + expf(-gsum))) * usum;
        hb[c][2 * wave + t] = h;
        if (H && c < mvalid) {
          const int64_t o = static_cast<int64_t>(col0 + c) * N + o0 + t;
          if constexpr (F16H) static_cast<uint16_t *>(H)[o] = static_cast<uint16_t>(f2h_bits(h));
          else static_cast<float *>(H)[o] = h;
        }
      }
  }
  if (Q) {
    __syncthreads();
    // whole groups of 8 lanes per batch column (quantizer shuffles stay inside)
    const int c = threadIdx.x >> 3, l = threadIdx.x & 7;
    if (c == 0 || c < mvalid) {  // mvalid >= 1
      const f32x4 h4 = *reinterpret_cast<const f32x4 *>(&hb[c][4 * l]);
      quantize4_store(h4.x, h4.y, h4.z, h4.w,
                      Q + (static_cast<int64_t>(col0 + c) * (N >> 5) + blockIdx.x) * kQ8_1Bytes, l);
    }
  }
}

// Q4_K with K <= 2048 and M <= 2: the same fusion on the wide slices of the
// grouped GEMV.  A row's K/64 <= 32 slices take half a wave, so a wave of a
// workgroup of NW waves computes 64 / NW rows (32 / NW per half) of one
// tensor: waves [0, NW/2) the 32 gate rows of the block, the others the 32
// up rows (the tensor is wave-uniform).  Lanes 31 and 63 put the row totals
// in LDS; after one barrier 8 lanes per batch column form h = silu(g) * u
// and quantize the block.  NORM = 1 / 2: the Q8_1 activations are produced
// in the kernel from an fp32 / fp16 residual (RMSNorm then Q8_1 by the first
// 256 threads, the standalone producer's arithmetic) into LDS, their loads
// issued before the weight prefetch.
struct SwigluArgs {
  const uint8_t *Wg, *Wu, *A;
  const void *x;
  const uint16_t *norm_w;
  float eps;
  void *H;
  uint8_t *Q;
  int M, N, K;
};

constexpr int kSwigluWideMaxK = 2048;

template <int MC, bool F16H, int NORM, int NW = 16>
__global__ __launch_bounds__(64 * NW) void k_gemv_swiglu_wide(const SwigluArgs args) {
  static_assert(NW == 4 || NW == 8 || NW == 16, "waves per workgroup");
  constexpr int kGW = NW / 2;   // waves per tensor
  constexpr int R = 32 / NW;    // rows per half-wave
  __shared__ float gu[2][MC][32];  // [gate/up][column][output]
  __shared__ __attribute__((aligned(16))) uint8_t a_lds[NORM ? MC * split_row_bytes(kSwigluWideMaxK) : 1];
  __shared__ float npart[4 * MC];
  [[maybe_unused]] constexpr int kStampBase = 2;
  IFX_STAMP(0);
  const int M = args.M, N = args.N, K = args.K;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const bool is_up = wave >= kGW;
  const int half = lane >> 5, lt = lane & 31;
  const int orow0 = ((wave % kGW) * 2 + half) * R;  // first output of this half-wave in the block
  const int col0 = blockIdx.y * MC;
  const int mvalid = min(MC, M - col0);
  const int nslice = K >> 6;
  const uint32_t a_row = static_cast<uint32_t>(K >> 5) * kQ8_1Bytes;
  const uint32_t w_row = static_cast<uint32_t>(row_bytes(kTypeQ4_K, K));
  const rsrc_t Wr = make_rsrc(is_up ? args.Wu : args.Wg, w_row * static_cast<uint32_t>(N));
  uint32_t voff[R], soff[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    voff[r] = static_cast<uint32_t>(blockIdx.x * 32 + orow0 + r) * w_row;
    soff[r] = 0u;
  }
  float acc[R][MC];
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int c = 0; c < MC; ++c) acc[r][c] = 0.0f;

  Q4Wide<R> wt;
  if constexpr (NORM != 0) {
    constexpr bool kXF16 = NORM == 2;
    const bool prod = threadIdx.x < 256;  // waves 0-3
    f32x4 xr[MC][2];
    u32x2 wr[MC][2];
    // every wave loads (the non-producer waves the producers' elements,
    // unused), so no branch surrounds the loads
#pragma unroll
    for (int c = 0; c < MC; ++c)
      rmsnorm_row_load_nb<kXF16, 2, true>(args.x, static_cast<int64_t>(col0 + min(c, mvalid - 1)) * K,
                                          args.norm_w, K, threadIdx.x, xr[c], wr[c]);
    // keep the activation loads ahead of the weight loads in issue order
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_sched_barrier(0);
    q4k_wide_load<R>(wt, Wr, voff, soff, min(lt, nslice - 1));  // unconditional (see above)
    if (prod) {
#pragma unroll
      for (int c = 0; c < MC; ++c)
        if (c < mvalid) rmsnorm_row_partial<2>(xr[c], K, npart + 4 * c, threadIdx.x);
    }
    __syncthreads();
    if (prod) {
#pragma unroll
      for (int c = 0; c < MC; ++c)
        if (c < mvalid)
          rmsnorm_row_apply<2, true>(xr[c], wr[c], a_lds + c * split_row_bytes(K), K, args.eps, npart + 4 * c,
                               threadIdx.x);
    }
    __syncthreads();
    IFX_STAMP(1);
    const ALdsS as{a_lds, static_cast<uint32_t>(split_row_bytes(K)), static_cast<uint32_t>(K / 64 * 80)};
    for (int s = lt; s < nslice; s += 32) {
      if (s != lt) q4k_wide_load<R>(wt, Wr, voff, soff, s);
      q4k_wide_compute<MC, R>(wt, as, mvalid, s, acc);
    }
  } else {
    const AGlobal as{make_rsrc(args.A + static_cast<int64_t>(col0) * a_row, a_row * mvalid), a_row};
    for (int s = lt; s < nslice; s += 32) {
      q4k_wide_load<R>(wt, Wr, voff, soff, s);
      q4k_wide_compute<MC, R>(wt, as, mvalid, s, acc);
    }
  }
  IFX_STAMP(2);
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int c = 0; c < MC; ++c) {
      const float v = halfwave_sum_to31(acc[r][c]);
      if (lt == 31) gu[is_up][c][orow0 + r] = v;
    }
  __syncthreads();
  IFX_STAMP(3);
  const int c = threadIdx.x >> 3, l = threadIdx.x & 7;
  if (c < MC && (c == 0 || c < mvalid)) {  // whole 8-lane groups (mvalid >= 1)
    const f32x4 g4 = *reinterpret_cast<const f32x4 *>(&gu[0][c][4 * l]);
    const f32x4 u4 = *reinterpret_cast<const f32x4 *>(&gu[1][c][4 * l]);
    const f32x4 h = silu_mul4(g4, u4);
    if (args.H) {
      const int64_t o = static_cast<int64_t>(col0 + c) * N + blockIdx.x * 32 + 4 * l;
      if constexpr (F16H) {
        const u32x2 hv = {f2h_bits(h.x) | (f2h_bits(h.y) << 16), f2h_bits(h.z) | (f2h_bits(h.w) << 16)};
        *reinterpret_cast<u32x2 *>(static_cast<uint16_t *>(args.H) + o) = hv;
      } else {
        *reinterpret_cast<f32x4 *>(static_cast<float *>(args.H) + o) = h;
      }
    }
    if (args.Q)
      quantize4_store(h.x, h.y, h.z, h.w,
                      args.Q + (static_cast<int64_t>(col0 + c) * (N >> 5) + blockIdx.x) * kQ8_1Bytes, l);
  }
}

// One workgroup per batch column (MC = 1 at M = 2 as well): the MC = 2 kernel
// needs 96 VGPRs, which leaves room for only one 16-wave workgroup per CU;
// the second column's weight reads mostly hit the cache.
template <int NORM, int NW>
static void launch_swiglu_wide_nw(const SwigluArgs &a, bool f16h, hipStream_t s) {
  const dim3 grid(a.N / 32, a.M);
  if (f16h) IFX_LAUNCH(k_gemv_swiglu_wide, (1, true, NORM, NW), grid, dim3(64 * NW), 0, s, a);
  else IFX_LAUNCH(k_gemv_swiglu_wide, (1, false, NORM, NW), grid, dim3(64 * NW), 0, s, a);
}
// Waves per workgroup, measured on MI355X (3B gate/up 11008 x 2048, cold
// weights, NW = 16 / 8 / 4): with the RMSNorm fused in 8 (M = 1: 8.4 / 8.1 /
// 8.7 us; M = 2: 10.8 / 10.2 / 10.5), from Q8_1 activations 16 (7.1 / 9.4 /
// 9.9 us).  IFX_SWIGLU_NW in {4, 8, 16} overrides (tuning; read once).
template <int NORM>
static void launch_swiglu_wide(const SwigluArgs &a, bool f16h, hipStream_t s) {
  static const int env = [] {
    const char *e = ifx::tuning_env("IFX_SWIGLU_NW");
    const int v = e ? atoi(e) : 0;
    return (v == 4 || v == 8 || v == 16) ? v : 0;
  }();
  const int nw = env ? env : NORM ? 8 : 16;
  if (nw == 4) launch_swiglu_wide_nw<NORM, 4>(a, f16h, s);
  else if (nw == 8) launch_swiglu_wide_nw<NORM, 8>(a, f16h, s);
  else launch_swiglu_wide_nw<NORM, 16>(a, f16h, s);
}

static bool swiglu_wide_env() {
  static const int v = [] {
    const char *e = ifx::tuning_env("IFX_SWIGLU_WIDE");
    return e ? atoi(e) : 1;
  }();
  return v != 0;
}

template <int QT, int MC>
static void launch_swiglu_mc(const uint8_t *Wg, const uint8_t *Wu, const uint8_t *A, void *H,
                             bool f16h, uint8_t *Q, int M, int N, int K, hipStream_t s) {
  const dim3 grid(N / 32, (M + MC - 1) / MC);
  if (f16h)
    IFX_LAUNCH(k_gemv_swiglu, (QT, MC, true), grid, dim3(1024), 0, s, Wg, Wu, A, H, Q, M, N, K);
  else
    IFX_LAUNCH(k_gemv_swiglu, (QT, MC, false), grid, dim3(1024), 0, s, Wg, Wu, A, H, Q, M, N, K);
}

template <int QT>
static void launch_swiglu_t(const uint8_t *Wg, const uint8_t *Wu, const uint8_t *A, void *H,
                            bool f16h, uint8_t *Q, int M, int N, int K, hipStream_t s) {
  if (M == 1) launch_swiglu_mc<QT, 1>(Wg, Wu, A, H, f16h, Q, M, N, K, s);
  else launch_swiglu_mc<QT, 2>(Wg, Wu, A, H, f16h, Q, M, N, K, s);
}

// 1 <= M <= 2, N % 32 == 0, K as for launch_gemv (checked by the caller).
hipError_t launch_gemv_swiglu(int qtype, const void *Wg, const void *Wu, const void *A, void *H,
                              bool f16h, void *Q, int M, int N, int K, hipStream_t stream) {
  const uint8_t *g = static_cast<const uint8_t *>(Wg), *u = static_cast<const uint8_t *>(Wu);
  const uint8_t *a = static_cast<const uint8_t *>(A);
  uint8_t *q = static_cast<uint8_t *>(Q);
  if (qtype == kTypeQ4_K && K <= kSwigluWideMaxK && M <= IFX_SWIGLU_MAX_M && swiglu_wide_env()) {
    const SwigluArgs args{g, u, a, nullptr, nullptr, 0.0f, H, q, M, N, K};
    launch_swiglu_wide<0>(args, f16h, stream);
    return last_error();
  }
  switch (qtype) {
  case kTypeQ4_K: launch_swiglu_t<kTypeQ4_K>(g, u, a, H, f16h, q, M, N, K, stream); break;
  case kTypeQ6_K: launch_swiglu_t<kTypeQ6_K>(g, u, a, H, f16h, q, M, N, K, stream); break;
  case kTypeQ8_0: launch_swiglu_t<kTypeQ8_0>(g, u, a, H, f16h, q, M, N, K, stream); break;
  case kTypeQ5_K: launch_swiglu_t<kTypeQ5_K>(g, u, a, H, f16h, q, M, N, K, stream); break;
  case kTypeQ8_K: launch_swiglu_t<kTypeQ8_K>(g, u, a, H, f16h, q, M, N, K, stream); break;
  default: return hipErrorInvalidValue;
  }
  return last_error();
}

// The wide Q4_K kernel with the RMSNorm + Q8_1 producer fused in (checked by
// the caller: Q4_K, K % 256 == 0, K <= 2048, 1 <= M <= 2, N % 32 == 0).
hipError_t launch_gemv_swiglu_rmsnorm(const void *Wg, const void *Wu, const void *x, bool x_f16,
                                      const uint16_t *norm_w, float eps, void *H, bool f16h,
                                      void *Q, int M, int N, int K, hipStream_t stream) {
  if (M < 1 || M > IFX_SWIGLU_MAX_M || K > kSwigluWideMaxK || N % 32 != 0) return hipErrorInvalidValue;
  const SwigluArgs args{static_cast<const uint8_t *>(Wg), static_cast<const uint8_t *>(Wu),
                        nullptr, x, norm_w, eps, H, static_cast<uint8_t *>(Q), M, N, K};
  if (x_f16) launch_swiglu_wide<2>(args, f16h, stream);
  else launch_swiglu_wide<1>(args, f16h, stream);
  return last_error();
}

// Geometry is validated by the caller: K % 256 == 0 for Q4_K/Q6_K,
// K % 32 == 0 for Q8_0, M >= 1, N >= 1.  M > 8 runs in groups of 8 columns
// (gridDim.y); the MFMA kernel covers large M.
hipError_t launch_gemv(int qtype, const void *W, const void *A, void *Y, const void *bias,
                       bool f16, int M, int N, int K, int mode, hipStream_t stream) {
  GemvArgs args{};
  args.seg[0] = GemvSeg{static_cast<const uint8_t *>(W), Y, bias, N, 0};
  args.nseg = 1;
  args.A = static_cast<const uint8_t *>(A);
  args.M = M;
  args.K = K;
  args.mode = mode;
  return launch_args(qtype, args, f16, stream);
}

// count (1..3) projections of one quant type over the same A, one launch.
hipError_t launch_gemv_grouped(int qtype, int count, const void *const *W, void *const *Y,
                               const int *N, const void *A, bool f16, int M, int K, int mode,
                               hipStream_t stream) {
  if (count < 1 || count > kMaxSeg) return hipErrorInvalidValue;
  GemvArgs args{};
  for (int i = 0; i < count; ++i)
    args.seg[i] = GemvSeg{static_cast<const uint8_t *>(W[i]), Y[i], nullptr, N[i], 0};
  args.nseg = count;
  args.A = static_cast<const uint8_t *>(A);
  args.M = M;
  args.K = K;
  args.mode = mode;
  return launch_args(qtype, args, f16, stream);
}

// The grouped Q4_K GEMV for 1 <= M <= 2 with the RMSNorm + Q8_1 producer
// fused in (checked by the caller: Q4_K, K % 256 == 0, M <= 2, the Q8_1
// copy of M rows fits 64 KiB of LDS).
hipError_t launch_gemv_rmsnorm(int count, const void *const *W, void *const *Y, const int *N,
                               const void *x, bool x_f16, const uint16_t *norm_w, float eps,
                               bool f16, int M, int K, int mode, hipStream_t stream) {
  // norm_w == nullptr: the plain quantizer
  if (count < 1 || count > kMaxSeg || M < 1 || M > 2) return hipErrorInvalidValue;
  GemvArgs args{};
  for (int i = 0; i < count; ++i)
    args.seg[i] = GemvSeg{static_cast<const uint8_t *>(W[i]), Y[i], nullptr, N[i], 0};
  args.nseg = count;
  args.A = nullptr;
  args.M = M;
  args.K = K;
  args.mode = mode;
  args.x = x;
  args.norm_w = norm_w;
  args.eps = eps;
  const int kind = (norm_w ? 1 : 3) + (x_f16 ? 1 : 0);
  if (M == 1) {
    switch (kind) {
    case 1: launch_norm_r<1, 1>(args, f16, stream); break;
    case 2: launch_norm_r<1, 2>(args, f16, stream); break;
    case 3: launch_norm_r<1, 3>(args, f16, stream); break;
    default: launch_norm_r<1, 4>(args, f16, stream); break;
    }
  } else {
    switch (kind) {
    case 1: launch_norm_r<2, 1>(args, f16, stream); break;
    case 2: launch_norm_r<2, 2>(args, f16, stream); break;
    case 3: launch_norm_r<2, 3>(args, f16, stream); break;
    default: launch_norm_r<2, 4>(args, f16, stream); break;
    }
  }
  return last_error();
}

}  // namespace ifx

#ifdef IFX_STAMPS
// Tuning builds: copies the wave timeline records of this file's kernels (8
// int64 per wave, see IFX_STAMP) to host memory, then clears them; returns
// the record count.
extern "C" int ifx_debug_stamps(long long *out, int max_waves) {
  const int n = max_waves < ifx::kStampWaves ? max_waves : ifx::kStampWaves;
  void *p = nullptr;
  if (hipGetSymbolAddress(&p, HIP_SYMBOL(ifx::ifx_stamps)) != hipSuccess) return -1;
  if (hipMemcpy(out, p, static_cast<size_t>(n) * 64, hipMemcpyDeviceToHost) != hipSuccess) return -1;
  if (hipMemset(p, 0, static_cast<size_t>(ifx::kStampWaves) * 64) != hipSuccess) return -1;
  return n;
}
#endif
