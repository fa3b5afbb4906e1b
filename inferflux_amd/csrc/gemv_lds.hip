// gemv_lds.hip -- Q4_K decode-batch GEMV for 3 <= M <= 8 with the Q8_1
// activations held in LDS: y[m][n] = sum_k W[n][k] * a[m][k].
//
// Same arithmetic as the M <= 2 GEMV and the reference's MMVQ kernels
// (runtime/backends/cuda/native/kernels/mmvq.cuh:49-158): an exact integer
// dot per 32-value sub-block, fp32 scaling by d*sc and the Q8_1 d, and the
// min term dmin*m times the Q8_1 s = d*sum(q) field (mmvq.cuh:115-125).
//
// Why a separate kernel.  The register-staged MFMA kernel (mmvq.hip) keeps
// one super-block per wave in flight and leaves its rescale work exposed;
// the M <= 2 GEMV streams weights at ~4 TB/s because every wave issues all
// its loads at once, but its lanes read the activations of every batch row
// from global memory (8 x 72 bytes per 36 weight bytes at M = 8).  Here a
// workgroup first copies the activations of all M rows into LDS once,
// de-interleaved -- int8 codes in 64-value slices padded to 80 bytes (lanes
// reading consecutive slices then hit distinct bank groups) and the d|s
// words in their own array -- and the waves then stream whole weight rows
// exactly as the M <= 2 GEMV does (one lane per 64 weights, wide slices),
// looping over the batch rows with their codes read from LDS.
//
// Limits: K % 256 == 0 and K <= 5120 (the LDS copy of A is M x K x 1.16
// bytes); the launcher routes other shapes elsewhere.
#include "ifx_common.h"

namespace ifx {

constexpr int kLdsSlicePitch = 80;  // 64 code bytes + 16 padding
constexpr int kLdsMaxK = 5120;

struct LdsSeg {
  const uint8_t *W;
  void *Y;
  const void *bias;
  int N;
  int blk_begin;
};

struct LdsArgs {
  LdsSeg seg[3];
  int nseg;
  const uint8_t *A;
  int M, K, mode;
};

// MC: largest M of the instantiation (4 or 8); R: rows per half-wave
// (H = 2, K <= 2048) or per wave (H = 1); P waves per workgroup.
template <int MC, int R, int H, int P, bool F16OUT>
__global__ __launch_bounds__(64 * P) void k_gemv_lds(const LdsArgs args) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const int M = args.M, K = args.K;
  const int nblk = K >> 5, nsl = K >> 6;  // Q8_1 blocks and 64-value slices per row
  const uint32_t code_row = static_cast<uint32_t>(nsl) * kLdsSlicePitch;
  uint8_t *codes = smem;                                        // [M][nsl][80]
  uint32_t *dsw = reinterpret_cast<uint32_t *>(smem + M * code_row);  // [M][nblk]

  // 1. weight rows; the first slice's loads go out before the activation
  // copy, so HBM latency overlaps it
  const int bx = blockIdx.x;
  const int si = (args.nseg > 2 && bx >= args.seg[2].blk_begin) ? 2
                 : (args.nseg > 1 && bx >= args.seg[1].blk_begin) ? 1 : 0;
  const LdsSeg &sg = args.seg[si];
  const int N = sg.N;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  constexpr int LPR = 64 / H;
  const int half = (H == 2) ? (lane >> 5) : 0;
  const int lt = lane & (LPR - 1);
  const int row0 = (((bx - sg.blk_begin) * P + wave) * H + half) * R;
  const uint32_t w_row = static_cast<uint32_t>(K >> 8) * kQ4KBytes;
  const rsrc_t Wr = make_rsrc(sg.W, w_row * static_cast<uint32_t>(N));
  uint32_t voff[R], soff[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const uint32_t ro = static_cast<uint32_t>(min(row0 + r, N - 1)) * w_row;
    voff[r] = (H == 2) ? ro : 0u;
    soff[r] = (H == 2) ? 0u : ro;
  }
  float acc[R][MC];
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int c = 0; c < MC; ++c) acc[r][c] = 0.0f;

  u32x4 hdr[R], q0[R], q1[R];
  auto load_w = [&](int s) {
    const int b = s >> 2, w = s & 3;
    const uint32_t wo = b * kQ4KBytes;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      hdr[r] = wload<u32x4>(Wr, voff[r] + wo, soff[r]);
      q0[r] = wload<u32x4>(Wr, voff[r] + wo + 16 + 32 * w, soff[r]);
      q1[r] = wload<u32x4>(Wr, voff[r] + wo + 32 + 32 * w, soff[r]);
    }
  };
  if (lt < nsl) load_w(lt);

  // 2. A -> LDS: one Q8_1 block (36 bytes) per thread and step
  {
    const rsrc_t Ag = make_rsrc(args.A, static_cast<uint32_t>(M * nblk) * kQ8_1Bytes);
    for (int j = threadIdx.x; j < M * nblk; j += 64 * P) {
      const int m = j / nblk, blk = j - m * nblk;
      const uint32_t go = static_cast<uint32_t>(j) * kQ8_1Bytes;
      const uint32_t ds = bload<uint32_t>(Ag, go, 0);
      const i32x4 c0 = bload<i32x4>(Ag, go + 4, 0);
      const i32x4 c1 = bload<i32x4>(Ag, go + 20, 0);
      uint8_t *dst = codes + m * code_row + (blk >> 1) * kLdsSlicePitch + (blk & 1) * 32;
      *reinterpret_cast<i32x4 *>(dst) = c0;
      *reinterpret_cast<i32x4 *>(dst + 16) = c1;
      dsw[j] = ds;
    }
  }
  __syncthreads();

  for (int s = lt; s < nsl; s += LPR) {
    const int w = s & 3;
    if (s != lt) load_w(s);
    // per row: the two sub-blocks' d*sc and dmin*m, and the 4-bit codes
    const int shift = 8 * ((2 * w) & 3);
    const uint32_t lo_mask = w < 2 ? 0x3F3F3F3Fu : 0x0F0F0F0Fu;
    const uint32_t top_mask = w < 2 ? 0u : 0x30303030u;
    float dsc0[R], dsc1[R], dm0[R], dm1[R];
    int lo[R][8], hi[R][8];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const float d = h2f(hdr[r].x & 0xFFFFu), dmin = h2f(hdr[r].x >> 16);
      const uint32_t S0 = hdr[r].y, S1 = hdr[r].z, S2 = hdr[r].w;
      const uint32_t scw = ((w < 2 ? S0 : S2) & lo_mask) | ((S0 >> 2) & top_mask);
      const uint32_t mw = ((w < 2 ? S1 : (S2 >> 4)) & lo_mask) | ((S1 >> 2) & top_mask);
      const uint32_t sct = scw >> shift, mt = mw >> shift;
      dsc0[r] = d * static_cast<float>(sct & 0xFFu);
      dsc1[r] = d * static_cast<float>((sct >> 8) & 0xFFu);
      dm0[r] = dmin * static_cast<float>(mt & 0xFFu);
      dm1[r] = dmin * static_cast<float>((mt >> 8) & 0xFFu);
      const uint32_t qv[8] = {q0[r].x, q0[r].y, q0[r].z, q0[r].w,
                              q1[r].x, q1[r].y, q1[r].z, q1[r].w};
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        lo[r][i] = static_cast<int>(qv[i] & 0x0F0F0F0Fu);
        hi[r][i] = static_cast<int>((qv[i] >> 4) & 0x0F0F0F0Fu);
      }
    }
    // batch rows: codes of Q8_1 blocks 8b + 2w (xa) and 8b + 2w + 1 (xb)
    // and their d|s words, from LDS
#pragma unroll
    for (int c = 0; c < MC; ++c) {
      if (c < M) {  // wave-uniform
        const uint8_t *cp = codes + c * code_row + s * kLdsSlicePitch;
        const i32x4 a0 = *reinterpret_cast<const i32x4 *>(cp);
        const i32x4 a1 = *reinterpret_cast<const i32x4 *>(cp + 16);
        const i32x4 b0 = *reinterpret_cast<const i32x4 *>(cp + 32);
        const i32x4 b1 = *reinterpret_cast<const i32x4 *>(cp + 48);
        const u32x2 dd = *reinterpret_cast<const u32x2 *>(dsw + c * nblk + 2 * s);
        const float da = h2f(dd.x & 0xFFFFu), sa = h2f(dd.x >> 16);
        const float db = h2f(dd.y & 0xFFFFu), sb = h2f(dd.y >> 16);
        const int xa[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
        const int xb[8] = {b0.x, b0.y, b0.z, b0.w, b1.x, b1.y, b1.z, b1.w};
#pragma unroll
        for (int r = 0; r < R; ++r) {
          int dl = 0, dh = 0;
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            dl = dot4(lo[r][i], xa[i], dl);
            dh = dot4(hi[r][i], xb[i], dh);
          }
          acc[r][c] += dsc0[r] * da * static_cast<float>(dl) +
                       dsc1[r] * db * static_cast<float>(dh) - (dm0[r] * sa + dm1[r] * sb);
        }
      }
    }
  }

  // 3. reduce over the lanes of each row set; lane 31 / 63 (H = 2) or 63
  // (H = 1) holds the totals
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int c = 0; c < MC; ++c)
      acc[r][c] = (H == 2) ? halfwave_sum_to31(acc[r][c]) : wave_sum_to63(acc[r][c]);
  if ((lane & (LPR - 1)) != LPR - 1) return;
  const int mode = args.mode;
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int row = row0 + r;
    if (row >= N) continue;
#pragma unroll
    for (int c = 0; c < MC; ++c) {
      if (c >= M) continue;
      float y = acc[r][c];
      const int64_t o = static_cast<int64_t>(c) * N + row;
      if constexpr (F16OUT) {
        uint16_t *Yh = static_cast<uint16_t *>(sg.Y);
        if (mode == 1) y += h2f(Yh[o]);
        else if (mode == 2) y += h2f(static_cast<const uint16_t *>(sg.bias)[row]);
        Yh[o] = static_cast<uint16_t>(f2h_bits(y));
      } else {
        float *Yf = static_cast<float *>(sg.Y);
        if (mode == 1) y += Yf[o];
        else if (mode == 2) y += static_cast<const float *>(sg.bias)[row];
        Yf[o] = y;
      }
    }
  }
}

namespace {

template <int MC, int R, int H, int P, bool F16>
void launch_lds_p(LdsArgs args, hipStream_t s) {
  int blocks = 0;
  for (int i = 0; i < args.nseg; ++i) {
    args.seg[i].blk_begin = blocks;
    const int rows_per_wg = P * H * R;
    blocks += (args.seg[i].N + rows_per_wg - 1) / rows_per_wg;
  }
  const int lds = args.M * ((args.K >> 6) * kLdsSlicePitch + (args.K >> 5) * 4);
  IFX_LAUNCH(k_gemv_lds, (MC, R, H, P, F16), dim3(blocks), dim3(64 * P), lds, s, args);
}

// Waves per workgroup: 8 (one activation copy per 32 rows at H = 2) unless
// that leaves fewer than ~512 workgroups, then 4 or 2.
template <int MC, int R, int H, bool F16>
void launch_lds_t(const LdsArgs &args, hipStream_t s) {
  int n_total = 0;
  for (int i = 0; i < args.nseg; ++i) n_total += args.seg[i].N;
  const int rows_per_wave = H * R;
  if (n_total >= 512 * 8 * rows_per_wave) launch_lds_p<MC, R, H, 8, F16>(args, s);
  else if (n_total >= 512 * 4 * rows_per_wave) launch_lds_p<MC, R, H, 4, F16>(args, s);
  else launch_lds_p<MC, R, H, 2, F16>(args, s);
}

template <int MC, bool F16>
void launch_lds_m(const LdsArgs &args, hipStream_t s) {
  if ((args.K >> 6) <= 32) launch_lds_t<MC, 2, 2, F16>(args, s);
  else launch_lds_t<MC, 2, 1, F16>(args, s);
}

}  // namespace

bool gemv_lds_fits(int qtype, int M, int K) {
  return qtype == kTypeQ4_K && M >= 1 && M <= 8 && K % 256 == 0 && K <= kLdsMaxK;
}

// count projections (1..3) of Q4_K sharing A; gemv_lds_fits() checked by
// the caller.  mode: 0 store, 1 accumulate, 2 bias (count == 1).
hipError_t launch_gemv_lds(int count, const void *const *W, void *const *Y, const int *N,
                           const void *bias, const void *A, bool f16, int M, int K, int mode,
                           hipStream_t stream) {
  if (count < 1 || count > 3) return hipErrorInvalidValue;
  LdsArgs args{};
  for (int i = 0; i < count; ++i)
    args.seg[i] = LdsSeg{static_cast<const uint8_t *>(W[i]), Y[i], i == 0 ? bias : nullptr, N[i], 0};
  args.nseg = count;
  args.A = static_cast<const uint8_t *>(A);
  args.M = M;
  args.K = K;
  args.mode = mode;
  if (M <= 4) {
    if (f16) launch_lds_m<4, true>(args, stream);
    else launch_lds_m<4, false>(args, stream);
  } else {
    if (f16) launch_lds_m<8, true>(args, stream);
    else launch_lds_m<8, false>(args, stream);
  }
  return last_error();
}

}  // namespace ifx
