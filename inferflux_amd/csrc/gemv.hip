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
//  * A "slice" is 32 weights of one row: 16 bytes of Q4_K qs (two half
//    sub-blocks), 16 bytes of Q6_K ql plus the matching 16 bytes of qh, or
//    one whole Q8_0 block.  A row has K/32 slices; lane l of a wave owns
//    slices l, l+64, ... of every row the wave visits.
//  * A wave owns R consecutive rows.  For each of its slices a lane loads
//    the activation codes and scales of all MC batch columns once into
//    registers and reuses them across the R rows, so activation traffic per
//    weight byte falls as 1/R.  Each weight byte is loaded exactly once,
//    with 16-byte loads whose lanes cover contiguous memory.
//  * Partial sums acc[R*MC] are combined across the 64 lanes with a
//    reduce-scatter butterfly (one shuffle per value per halving step), so
//    lane i ends with one finished output instead of all lanes reducing all
//    values.
// No LDS, no barriers: waves are independent and exit on their own.
#include "ifx_common.h"

namespace ifx {

enum OutMode { kOutStore = 0, kOutAccum = 1, kOutBias = 2 };

// Activation view of one slice for one batch column.
struct ActQ4 {  // Q4_K: half sub-blocks 2p and 2p+1
  int xa[4], xb[4];
  float da, db, sa, sb;
};

template <int QT>
__device__ __forceinline__ int slices_per_row(int K) {
  return K >> 5;
}

// ---------------------------------------------------------------------------
// Per-type slice kernels.  Each computes, for one slice and one row, the
// contribution to acc[0..MC-1] given that slice's activations.
// ---------------------------------------------------------------------------

template <int MC, int R>
__device__ __forceinline__ void q4k_slices(const uint8_t *__restrict__ W,
                                           const uint8_t *__restrict__ A, int row0, int N,
                                           int K, int mvalid, int lane, float (&acc)[R][MC]) {
  const int nsb = K >> 8;
  const int nslice = K >> 5;
  const int64_t a_row = static_cast<int64_t>(K >> 5) * kQ8_1Bytes;
  for (int s = lane; s < nslice; s += kWave) {
    const int b = s >> 3, j = s & 7, p = j >> 1, h = j & 1;
    // Activations: Q8_1 blocks (b*8 + 2p) and (b*8 + 2p + 1), bytes 16h..16h+15.
    int xa[MC][4], xb[MC][4];
    float da[MC], db[MC], sa[MC], sbv[MC];
#pragma unroll
    for (int c = 0; c < MC; ++c) {
      if (c < mvalid) {
        const uint8_t *ab = A + c * a_row + static_cast<int64_t>(b * 8 + 2 * p) * kQ8_1Bytes;
        const uint32_t dsa = ldg<uint32_t>(ab);
        const uint32_t dsb = ldg<uint32_t>(ab + kQ8_1Bytes);
        const i32x4 va = ldg<i32x4>(ab + 4 + 16 * h);
        const i32x4 vb = ldg<i32x4>(ab + kQ8_1Bytes + 4 + 16 * h);
        xa[c][0] = va.x; xa[c][1] = va.y; xa[c][2] = va.z; xa[c][3] = va.w;
        xb[c][0] = vb.x; xb[c][1] = vb.y; xb[c][2] = vb.z; xb[c][3] = vb.w;
        da[c] = h2f(dsa & 0xFFFFu);
        db[c] = h2f(dsb & 0xFFFFu);
        // The min term is per 32-value sub-block: only the h == 0 lane adds it.
        sa[c] = h ? 0.0f : h2f(dsa >> 16);
        sbv[c] = h ? 0.0f : h2f(dsb >> 16);
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) xa[c][i] = xb[c][i] = 0;
        da[c] = db[c] = sa[c] = sbv[c] = 0.0f;
      }
    }
    const int shift = 8 * ((2 * p) & 3);
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int row = row0 + r;
      if (row >= N) break;
      const uint8_t *blk = W + (static_cast<int64_t>(row) * nsb + b) * kQ4KBytes;
      const u32x4 hdr = ldg<u32x4>(blk);
      const u32x4 q = ldg<u32x4>(blk + 16 + 16 * j);
      const float d = h2f(hdr.x & 0xFFFFu);
      const float dmin = h2f(hdr.x >> 16);
      // 6-bit scale/min unpack (quant_common.cuh:83-94) for all 8 sub-blocks
      // at once, 4 per dword: sub-blocks 0-3 and 4-7.
      const uint32_t S0 = hdr.y, S1 = hdr.z, S2 = hdr.w;
      const uint32_t sc_lo4 = S0 & 0x3F3F3F3Fu;
      const uint32_t m_lo4 = S1 & 0x3F3F3F3Fu;
      const uint32_t sc_hi4 = (S2 & 0x0F0F0F0Fu) | ((S0 >> 2) & 0x30303030u);
      const uint32_t m_hi4 = ((S2 >> 4) & 0x0F0F0F0Fu) | ((S1 >> 2) & 0x30303030u);
      const uint32_t scw = (p < 2) ? sc_lo4 : sc_hi4;
      const uint32_t mw = (p < 2) ? m_lo4 : m_hi4;
      const float sc0 = static_cast<float>((scw >> shift) & 0xFFu);
      const float sc1 = static_cast<float>((scw >> (shift + 8)) & 0xFFu);
      const float m0 = static_cast<float>((mw >> shift) & 0xFFu);
      const float m1 = static_cast<float>((mw >> (shift + 8)) & 0xFFu);
      const float dsc0 = d * sc0, dsc1 = d * sc1, dm0 = dmin * m0, dm1 = dmin * m1;
      int lo[4], hi[4];
      lo[0] = q.x & 0x0F0F0F0F; hi[0] = (q.x >> 4) & 0x0F0F0F0F;
      lo[1] = q.y & 0x0F0F0F0F; hi[1] = (q.y >> 4) & 0x0F0F0F0F;
      lo[2] = q.z & 0x0F0F0F0F; hi[2] = (q.z >> 4) & 0x0F0F0F0F;
      lo[3] = q.w & 0x0F0F0F0F; hi[3] = (q.w >> 4) & 0x0F0F0F0F;
#pragma unroll
      for (int c = 0; c < MC; ++c) {
        int dl = 0, dh = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          dl = dot4(lo[i], xa[c][i], dl);
          dh = dot4(hi[i], xb[c][i], dh);
        }
        acc[r][c] += dsc0 * da[c] * static_cast<float>(dl) + dsc1 * db[c] * static_cast<float>(dh) -
                     (dm0 * sa[c] + dm1 * sbv[c]);
      }
    }
  }
}

template <int MC, int R>
__device__ __forceinline__ void q6k_slices(const uint8_t *__restrict__ W,
                                           const uint8_t *__restrict__ A, int row0, int N,
                                           int K, int mvalid, int lane, float (&acc)[R][MC]) {
  const int nsb = K >> 8;
  const int nslice = K >> 5;
  const int64_t a_row = static_cast<int64_t>(K >> 5) * kQ8_1Bytes;
  for (int s = lane; s < nslice; s += kWave) {
    // Slice j of super-block b: group g, ql half c (sub-blocks c and c+2),
    // element half h (values 16h..16h+15 of each sub-block).
    const int b = s >> 3, j = s & 7, g = j >> 2, cc = (j >> 1) & 1, h = j & 1;
    int xa[MC][4], xb[MC][4];
    float da[MC], db[MC];
    int suma[MC], sumb[MC];
#pragma unroll
    for (int c = 0; c < MC; ++c) {
      if (c < mvalid) {
        const uint8_t *ab = A + c * a_row + static_cast<int64_t>(b * 8 + g * 4 + cc) * kQ8_1Bytes;
        const uint8_t *bb = ab + 2 * kQ8_1Bytes;
        const i32x4 va = ldg<i32x4>(ab + 4 + 16 * h);
        const i32x4 vb = ldg<i32x4>(bb + 4 + 16 * h);
        xa[c][0] = va.x; xa[c][1] = va.y; xa[c][2] = va.z; xa[c][3] = va.w;
        xb[c][0] = vb.x; xb[c][1] = vb.y; xb[c][2] = vb.z; xb[c][3] = vb.w;
        da[c] = h2f(ldg<uint16_t>(ab));
        db[c] = h2f(ldg<uint16_t>(bb));
        // sum of the activation codes, for the -32 offset of Q6_K codes
        int s0 = 0, s1 = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          s0 = dot4(0x01010101, xa[c][i], s0);
          s1 = dot4(0x01010101, xb[c][i], s1);
        }
        suma[c] = 32 * s0;
        sumb[c] = 32 * s1;
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) xa[c][i] = xb[c][i] = 0;
        da[c] = db[c] = 0.0f;
        suma[c] = sumb[c] = 0;
      }
    }
    const int sh_a = 2 * cc, sh_b = 2 * cc + 4;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int row = row0 + r;
      if (row >= N) break;
      const uint8_t *blk = W + (static_cast<int64_t>(row) * nsb + b) * kQ6KBytes;
      const u32x4 ql = ldg<u32x4>(blk + g * 64 + cc * 32 + 16 * h);
      const u32x4 qh = ldg<u32x4>(blk + 128 + g * 32 + 16 * h);
      const u32x2 scw = ldg<u32x2>(blk + 192 + g * 8);
      const float d = h2f(ldg<uint16_t>(blk + 208));
      // scales[g*8 + 2*sub + h] for sub = cc (dword 0) and sub = cc + 2 (dword 1)
      const int sca = static_cast<int8_t>((scw.x >> (8 * (2 * cc + h))) & 0xFFu);
      const int scb = static_cast<int8_t>((scw.y >> (8 * (2 * cc + h))) & 0xFFu);
      const float dsa = d * static_cast<float>(sca), dsb = d * static_cast<float>(scb);
      const uint32_t qlv[4] = {ql.x, ql.y, ql.z, ql.w};
      const uint32_t qhv[4] = {qh.x, qh.y, qh.z, qh.w};
      int va[4], vb[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        va[i] = static_cast<int>((qlv[i] & 0x0F0F0F0Fu) | (((qhv[i] >> sh_a) & 0x03030303u) << 4));
        vb[i] = static_cast<int>(((qlv[i] >> 4) & 0x0F0F0F0Fu) | (((qhv[i] >> sh_b) & 0x03030303u) << 4));
      }
#pragma unroll
      for (int c = 0; c < MC; ++c) {
        int dA = 0, dB = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          dA = dot4(va[i], xa[c][i], dA);
          dB = dot4(vb[i], xb[c][i], dB);
        }
        dA -= suma[c];
        dB -= sumb[c];
        acc[r][c] += dsa * da[c] * static_cast<float>(dA) + dsb * db[c] * static_cast<float>(dB);
      }
    }
  }
}

template <int MC, int R>
__device__ __forceinline__ void q8_0_slices(const uint8_t *__restrict__ W,
                                            const uint8_t *__restrict__ A, int row0, int N,
                                            int K, int mvalid, int lane, float (&acc)[R][MC]) {
  const int nblk = K >> 5;
  const int64_t a_row = static_cast<int64_t>(nblk) * kQ8_1Bytes;
  for (int s = lane; s < nblk; s += kWave) {
    int x[MC][8];
    float da[MC];
#pragma unroll
    for (int c = 0; c < MC; ++c) {
      if (c < mvalid) {
        const uint8_t *ab = A + c * a_row + static_cast<int64_t>(s) * kQ8_1Bytes;
        const i32x4 v0 = ldg<i32x4>(ab + 4);
        const i32x4 v1 = ldg<i32x4>(ab + 20);
        x[c][0] = v0.x; x[c][1] = v0.y; x[c][2] = v0.z; x[c][3] = v0.w;
        x[c][4] = v1.x; x[c][5] = v1.y; x[c][6] = v1.z; x[c][7] = v1.w;
        da[c] = h2f(ldg<uint16_t>(ab));
      } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) x[c][i] = 0;
        da[c] = 0.0f;
      }
    }
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int row = row0 + r;
      if (row >= N) break;
      const uint8_t *blk = W + (static_cast<int64_t>(row) * nblk + s) * kQ8_0Bytes;
      const float d = h2f(ldg<uint16_t>(blk));
      const i32x4 w0 = ldg<i32x4>(blk + 2);
      const i32x4 w1 = ldg<i32x4>(blk + 18);
      const int wv[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
#pragma unroll
      for (int c = 0; c < MC; ++c) {
        int dt = 0;
#pragma unroll
        for (int i = 0; i < 8; ++i) dt = dot4(wv[i], x[c][i], dt);
        acc[r][c] += d * da[c] * static_cast<float>(dt);
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Kernel: one wave per R rows; blockIdx.y selects the group of MC columns.
// ---------------------------------------------------------------------------
template <int QT, int MC, int R, bool F16OUT>
__global__ __launch_bounds__(256) void k_gemv(const uint8_t *__restrict__ W,
                                              const uint8_t *__restrict__ A,
                                              void *__restrict__ Y, const void *__restrict__ bias,
                                              int M, int N, int K, int mode) {
  const int lane = threadIdx.x & 63;
  const int wave = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int row0 = wave * R;
  if (row0 >= N) return;
  const int col0 = blockIdx.y * MC;
  const int mvalid = min(MC, M - col0);
  const uint8_t *Ac = A + static_cast<int64_t>(col0) * (K >> 5) * kQ8_1Bytes;

  float acc[R][MC];
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int c = 0; c < MC; ++c) acc[r][c] = 0.0f;

  if constexpr (QT == kTypeQ4_K)
    q4k_slices<MC, R>(W, Ac, row0, N, K, mvalid, lane, acc);
  else if constexpr (QT == kTypeQ6_K)
    q6k_slices<MC, R>(W, Ac, row0, N, K, mvalid, lane, acc);
  else
    q8_0_slices<MC, R>(W, Ac, row0, N, K, mvalid, lane, acc);

  // Reduce-scatter over the wave.  V = R*MC values, V a power of two <= 64.
  constexpr int V = R * MC;
  float v[V];
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int c = 0; c < MC; ++c) v[r * MC + c] = acc[r][c];
  // Halving steps with lane offsets 32, 16, ...: after the step with offset o
  // and length L, a lane with (lane & o) keeps the upper half.
  int o = 32;
#pragma unroll
  for (int L = V; L > 1; L >>= 1, o >>= 1) {
    const bool up = (lane & o) != 0;
#pragma unroll
    for (int i = 0; i < L / 2; ++i) {
      const float send = up ? v[i] : v[i + L / 2];
      const float keep = up ? v[i + L / 2] : v[i];
      v[i] = keep + __shfl_xor(send, o);
    }
  }
  for (; o >= 1; o >>= 1) v[0] += __shfl_xor(v[0], o);
  // Lane index bits 5, 4, ... (high first) encode the kept value index.
  constexpr int kLowBits = 6 - __builtin_ctz(V);  // bits below the index bits
  if ((lane & ((1 << kLowBits) - 1)) != 0) return;
  const int idx = lane >> kLowBits;
  // The value index built from lane bits: bit5 selects V/2, bit4 V/4, ...
  // so idx read high-to-low is the index itself.
  const int r = idx / MC, c = idx % MC;
  const int row = row0 + r;
  if (row >= N || c >= mvalid) return;
  const int64_t o_idx = static_cast<int64_t>(col0 + c) * N + row;
  float y = v[0];
  if constexpr (F16OUT) {
    uint16_t *Yh = static_cast<uint16_t *>(Y);
    if (mode == kOutAccum) y += h2f(Yh[o_idx]);
    else if (mode == kOutBias) y += h2f(static_cast<const uint16_t *>(bias)[row]);
    Yh[o_idx] = static_cast<uint16_t>(f2h_bits(y));
  } else {
    float *Yf = static_cast<float *>(Y);
    if (mode == kOutAccum) y += Yf[o_idx];
    else if (mode == kOutBias) y += static_cast<const float *>(bias)[row];
    Yf[o_idx] = y;
  }
}

template <int QT, int MC, int R>
static void launch_t(const uint8_t *W, const uint8_t *A, void *Y, const void *bias, bool f16,
                     int M, int N, int K, int mode, hipStream_t s) {
  const int waves = (N + R - 1) / R;
  const dim3 grid((waves + 3) / 4, (M + MC - 1) / MC);
  if (f16)
    hipLaunchKernelGGL((k_gemv<QT, MC, R, true>), grid, dim3(256), 0, s, W, A, Y, bias, M, N, K, mode);
  else
    hipLaunchKernelGGL((k_gemv<QT, MC, R, false>), grid, dim3(256), 0, s, W, A, Y, bias, M, N, K, mode);
}

template <int QT>
static void launch_type(const uint8_t *W, const uint8_t *A, void *Y, const void *bias, bool f16,
                        int M, int N, int K, int mode, hipStream_t s) {
  if (M == 1) launch_t<QT, 1, 8>(W, A, Y, bias, f16, M, N, K, mode, s);
  else if (M == 2) launch_t<QT, 2, 8>(W, A, Y, bias, f16, M, N, K, mode, s);
  else if (M <= 4) launch_t<QT, 4, 4>(W, A, Y, bias, f16, M, N, K, mode, s);
  else launch_t<QT, 8, 4>(W, A, Y, bias, f16, M, N, K, mode, s);
}

// Geometry is validated by the caller: K % 256 == 0 for Q4_K/Q6_K,
// K % 32 == 0 for Q8_0, M >= 1, N >= 1.  M > 8 runs in groups of 8 columns
// (gridDim.y); the MFMA kernel covers large M.
hipError_t launch_gemv(int qtype, const void *W, const void *A, void *Y, const void *bias,
                       bool f16, int M, int N, int K, int mode, hipStream_t stream) {
  const uint8_t *w = static_cast<const uint8_t *>(W);
  const uint8_t *a = static_cast<const uint8_t *>(A);
  switch (qtype) {
  case kTypeQ4_K: launch_type<kTypeQ4_K>(w, a, Y, bias, f16, M, N, K, mode, stream); break;
  case kTypeQ6_K: launch_type<kTypeQ6_K>(w, a, Y, bias, f16, M, N, K, mode, stream); break;
  case kTypeQ8_0: launch_type<kTypeQ8_0>(w, a, Y, bias, f16, M, N, K, mode, stream); break;
  default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace ifx
