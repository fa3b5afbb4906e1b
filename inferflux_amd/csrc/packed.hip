// packed.hip -- GEMV on per-row symmetric int8 activations (the
// reference's packed-activation path, FusedQuantGemm::GemvPacked /
// GemvPackedPair / GemvPackedTriple, fused_quant_gemm.h:79-107 and .cu
// 1131-1231; kernels fused_dequant_gemv.cuh:80-580).
//
// y[m][n] = fp16( scale[m] * sum_k W[n][k] * q[m][k] ), W raw GGUF Q4_K,
// Q6_K, Q8_0 or Q8_K, q the int8 codes of ifx_quantize_rows_symmetric with
// one fp32 scale per batch row.  Per weight block the integer dot products
// are exact (v_dot4_i32_i8); the block's float scales apply in fp32:
//   Q4_K  d*sc*dot(q4, x) - dmin*m*sum(x)      per 32-value sub-block
//   Q6_K  d*sc*(dot(q6u, x) - 32*sum(x))       per 16 values (q6u = q + 32)
//   Q8_0  d*dot(q, x)                          per 32 values
//   Q8_K  d*dot(q, x)                          per 64 values (d fp32)
// and the row scale once per output.  The reference sums the same terms
// with the row scale inside every block, so results differ by rounding.
//
// Mapping: the M <= 2 GEMV's wide slices.  A lane takes 64 consecutive
// values of a row (32 for Q8_0: one block), 16-byte weight and activation
// loads through buffer resources; a row of at most 32 slices is half a wave
// (two rows per wave), longer rows a full wave.  Four waves per workgroup;
// blockIdx.y selects MC batch rows, so each weight byte is read ceil(M / MC)
// times.  blockIdx.x walks the row groups of up to three projections that
// share the activations (pair / triple).
#include "ifx_common.h"

namespace ifx {

namespace {

struct PackedSeg {
  const uint8_t *W;
  uint16_t *Y;
  int N;
  int blk_begin;
};
struct PackedArgs {
  PackedSeg seg[3];
  int nseg;
  const int8_t *X;
  const float *scales;
  int M, K;
};

constexpr int kWaves = 4;

template <int QT>
constexpr int slice_values() { return QT == kTypeQ8_0 ? 32 : 64; }

// One slice of one row times MC activation rows; adds the unscaled
// (row-scale-free) block sums into acc[c].
template <int QT, int MC>
__device__ __forceinline__ void packed_slice(rsrc_t Wr, uint32_t row_off, rsrc_t Xr,
                                             uint32_t x_row, int mvalid, int s, float (&acc)[MC]) {
  if constexpr (QT == kTypeQ4_K) {
    // super-block b, sub-blocks 2p (low nibbles) and 2p + 1 (high nibbles)
    const int b = s >> 2, p = s & 3;
    const uint32_t wo = row_off + b * kQ4KBytes;
    const u32x4 hdr = wload<u32x4>(Wr, wo, 0);
    const u32x4 q0 = wload<u32x4>(Wr, wo + 16 + 32 * p, 0);
    const u32x4 q1 = wload<u32x4>(Wr, wo + 32 + 32 * p, 0);
    i32x4 xl0[MC], xl1[MC], xh0[MC], xh1[MC];
    const uint32_t xo = b * 256 + 64 * p;
#pragma unroll
    for (int c = 0; c < MC; ++c) {
      const uint32_t o = xo + (c < mvalid ? c : 0) * x_row;
      xl0[c] = bload<i32x4>(Xr, o, 0);
      xl1[c] = bload<i32x4>(Xr, o + 16, 0);
      xh0[c] = bload<i32x4>(Xr, o + 32, 0);
      xh1[c] = bload<i32x4>(Xr, o + 48, 0);
    }
    // get_scale_min_k4 (quant_common.cuh:83-94) for j = 2p and 2p + 1:
    // bytes 0-3 of the 12 scale bytes (words S0, S1, S2 = header words 1-3)
    // hold the 6-bit scales of j < 4, bytes 4-7 their mins; j >= 4 take the
    // low / high nibble of bytes 8-11 and the top two bits of bytes 0-7
    const float d = h2f(hdr.x & 0xFFFFu), dmin = h2f(hdr.x >> 16);
    const uint32_t S0 = hdr.y, S1 = hdr.z, S2 = hdr.w;
    const bool lo = p < 2;
    const uint32_t scw = lo ? (S0 & 0x3F3F3F3Fu) : ((S2 & 0x0F0F0F0Fu) | ((S0 >> 2) & 0x30303030u));
    const uint32_t mw = lo ? (S1 & 0x3F3F3F3Fu) : (((S2 >> 4) & 0x0F0F0F0Fu) | ((S1 >> 2) & 0x30303030u));
    const int sh = 16 * (p & 1);
    const float dsc0 = d * static_cast<float>((scw >> sh) & 0xFFu);
    const float dsc1 = d * static_cast<float>((scw >> (sh + 8)) & 0xFFu);
    const float dm0 = dmin * static_cast<float>((mw >> sh) & 0xFFu);
    const float dm1 = dmin * static_cast<float>((mw >> (sh + 8)) & 0xFFu);
    const uint32_t qv[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
#pragma unroll
    for (int c = 0; c < MC; ++c) {
      const int xl[8] = {xl0[c].x, xl0[c].y, xl0[c].z, xl0[c].w, xl1[c].x, xl1[c].y, xl1[c].z, xl1[c].w};
      const int xh[8] = {xh0[c].x, xh0[c].y, xh0[c].z, xh0[c].w, xh1[c].x, xh1[c].y, xh1[c].z, xh1[c].w};
      int dl = 0, dh = 0, sl = 0, shs = 0;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        dl = dot4(static_cast<int>(qv[i] & 0x0F0F0F0Fu), xl[i], dl);
        dh = dot4(static_cast<int>((qv[i] >> 4) & 0x0F0F0F0Fu), xh[i], dh);
        sl = dot4(0x01010101, xl[i], sl);
        shs = dot4(0x01010101, xh[i], shs);
      }
      acc[c] += (dsc0 * static_cast<float>(dl) - dm0 * static_cast<float>(sl)) +
                (dsc1 * static_cast<float>(dh) - dm1 * static_cast<float>(shs));
    }
  } else if constexpr (QT == kTypeQ6_K) {
    // dequant_q6k_element (quant_common.cuh:161-177): slice s covers, in
    // 128-value half g of super-block b, the values 32k + 16h + (0..15) for
    // k = 0..3 (ql bytes 16h.. and 32 + 16h.. of the half, qh bytes 16h..)
    const int b = s >> 2, g = (s >> 1) & 1, h = s & 1;
    const uint32_t wo = row_off + b * kQ6KBytes;
    const u32x4 ql0 = wload<u32x4>(Wr, wo + g * 64 + 16 * h, 0);
    const u32x4 ql1 = wload<u32x4>(Wr, wo + g * 64 + 32 + 16 * h, 0);
    const u32x4 qh = wload<u32x4>(Wr, wo + 128 + g * 32 + 16 * h, 0);
    const u32x2 scw = wload<u32x2>(Wr, wo + 192 + g * 8, 0);
    const uint32_t db = wload<uint16_t>(Wr, wo + 208, 0);
    i32x4 x[4][MC];
    const uint32_t xo = b * 256 + g * 128 + 16 * h;
#pragma unroll
    for (int c = 0; c < MC; ++c)
#pragma unroll
      for (int k = 0; k < 4; ++k) x[k][c] = bload<i32x4>(Xr, xo + 32 * k + (c < mvalid ? c : 0) * x_row, 0);
    const float d = h2f(db);
    // scales[8g + 2k + h]: dword 0 of the group's 8 bytes holds k = 0, 1
    // (bytes h, h + 2), dword 1 k = 2, 3
    const int ss = 8 * h;
    float dsk[4];
    dsk[0] = d * static_cast<float>(static_cast<int8_t>((scw.x >> ss) & 0xFFu));
    dsk[1] = d * static_cast<float>(static_cast<int8_t>((scw.x >> (ss + 16)) & 0xFFu));
    dsk[2] = d * static_cast<float>(static_cast<int8_t>((scw.y >> ss) & 0xFFu));
    dsk[3] = d * static_cast<float>(static_cast<int8_t>((scw.y >> (ss + 16)) & 0xFFu));
    const uint32_t l0[4] = {ql0.x, ql0.y, ql0.z, ql0.w};
    const uint32_t l1[4] = {ql1.x, ql1.y, ql1.z, ql1.w};
    const uint32_t hv[4] = {qh.x, qh.y, qh.z, qh.w};
    int v[4][4];
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
        const int xs[4] = {x[k][c].x, x[k][c].y, x[k][c].z, x[k][c].w};
        int dt = 0, sx = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          dt = dot4(v[k][i], xs[i], dt);
          sx = dot4(0x01010101, xs[i], sx);
        }
        sum += dsk[k] * static_cast<float>(dt - 32 * sx);
      }
      acc[c] += sum;
    }
  } else if constexpr (QT == kTypeQ8_0) {
    // dequant_q8_0_element (quant_common.cuh:185-188): block s, 34 bytes
    const uint32_t wo = row_off + s * kQ8_0Bytes;
    const uint32_t db = wload<uint16_t>(Wr, wo, 0);
    const u32x4 q0 = wload<u32x4>(Wr, wo + 2, 0);
    const u32x4 q1 = wload<u32x4>(Wr, wo + 18, 0);
    const float d = h2f(db);
    const uint32_t qv[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
#pragma unroll
    for (int c = 0; c < MC; ++c) {
      const uint32_t o = s * 32 + (c < mvalid ? c : 0) * x_row;
      const i32x4 x0 = bload<i32x4>(Xr, o, 0), x1 = bload<i32x4>(Xr, o + 16, 0);
      const int xs[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
      int dt = 0;
#pragma unroll
      for (int i = 0; i < 8; ++i) dt = dot4(static_cast<int>(qv[i]), xs[i], dt);
      acc[c] += d * static_cast<float>(dt);
    }
  } else {
    // Q8_K (quant_common.cuh block_q8_k): fp32 d, 256 int8 codes, bsums;
    // slice s = 64 codes of super-block s / 4
    const int b = s >> 2, p = s & 3;
    const uint32_t wo = row_off + b * kQ8KBytes;
    const float d = __builtin_bit_cast(float, wload<uint32_t>(Wr, wo, 0));
    u32x4 q[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) q[i] = wload<u32x4>(Wr, wo + 4 + 64 * p + 16 * i, 0);
#pragma unroll
    for (int c = 0; c < MC; ++c) {
      const uint32_t o = b * 256 + 64 * p + (c < mvalid ? c : 0) * x_row;
      int dt = 0;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const i32x4 x = bload<i32x4>(Xr, o + 16 * i, 0);
        dt = dot4(static_cast<int>(q[i].x), x.x, dt);
        dt = dot4(static_cast<int>(q[i].y), x.y, dt);
        dt = dot4(static_cast<int>(q[i].z), x.z, dt);
        dt = dot4(static_cast<int>(q[i].w), x.w, dt);
      }
      acc[c] += d * static_cast<float>(dt);
    }
  }
}

}  // namespace

// H = 2 / 4: two / four rows per wave (32 / 16 lanes each); H = 1: one row
// per wave.
template <int QT, int MC, int H>
__global__ __launch_bounds__(64 * kWaves) void k_gemv_packed(const PackedArgs args) {
  constexpr int LPR = 64 / H;  // lanes per row
  const int bx = blockIdx.x;
  const bool in2 = args.nseg > 2 && bx >= args.seg[2].blk_begin;
  const bool in1 = !in2 && args.nseg > 1 && bx >= args.seg[1].blk_begin;
  const PackedSeg sg = in2 ? args.seg[2] : in1 ? args.seg[1] : args.seg[0];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int half = lane / LPR, lt = lane & (LPR - 1);  // row of the wave, lane in it
  const int n = ((bx - sg.blk_begin) * kWaves + wave) * H + half;
  const int N = sg.N, M = args.M, K = args.K;
  const int col0 = blockIdx.y * MC;
  const int mvalid = min(MC, M - col0);
  const uint32_t w_row = static_cast<uint32_t>(row_bytes(QT, K));
  const rsrc_t Wr = make_rsrc(sg.W, w_row * static_cast<uint32_t>(N));
  const rsrc_t Xr = make_rsrc(args.X + static_cast<int64_t>(col0) * K,
                              static_cast<uint32_t>(K) * static_cast<uint32_t>(mvalid));
  const uint32_t row_off = static_cast<uint32_t>(min(n, N - 1)) * w_row;
  const int nslice = K / slice_values<QT>();

  float acc[MC];
#pragma unroll
  for (int c = 0; c < MC; ++c) acc[c] = 0.0f;
  for (int s = lt; s < nslice; s += LPR)
    packed_slice<QT, MC>(Wr, row_off, Xr, static_cast<uint32_t>(K), mvalid, s, acc);

  float tot[MC];
#pragma unroll
  for (int c = 0; c < MC; ++c)
    tot[c] = H == 4 ? quarterwave_sum(acc[c]) : H == 2 ? halfwave_sum_to31(acc[c]) : wave_sum_to63(acc[c]);
  if (lt != LPR - 1 || n >= N) return;
#pragma unroll
  for (int c = 0; c < MC; ++c)
    if (c < mvalid) {
      const int m = col0 + c;
      sg.Y[static_cast<int64_t>(m) * N + n] =
          static_cast<uint16_t>(f2h_bits(tot[c] * args.scales[m]));
    }
}

namespace {

// Rows per wave: half-wave rows for at most 32 slices; quarter-wave rows
// when 16 lanes leave none idle and a full wave would (K = 5120: 80 slices,
// 5 per lane); else full-wave rows.
int rows_per_wave(int nslice) {
  if (nslice <= 32) return 2;
  if (nslice % 16 == 0 && nslice % 64 != 0 && nslice <= 128) return 4;
  return 1;
}

template <int QT, int MC>
hipError_t launch_mc(const PackedArgs &args, int groups, int H, hipStream_t s) {
  const dim3 block(64 * kWaves), grid(groups, (args.M + MC - 1) / MC);
  if (H == 4) IFX_LAUNCH(k_gemv_packed, (QT, MC, 4), grid, block, 0, s, args);
  else if (H == 2) IFX_LAUNCH(k_gemv_packed, (QT, MC, 2), grid, block, 0, s, args);
  else IFX_LAUNCH(k_gemv_packed, (QT, MC, 1), grid, block, 0, s, args);
  return last_error();
}

template <int QT>
hipError_t launch_qt(PackedArgs args, hipStream_t s) {
  // row groups: kWaves * H rows per workgroup
  const int H = rows_per_wave(args.K / slice_values<QT>());
  int groups = 0;
  for (int i = 0; i < args.nseg; ++i) {
    args.seg[i].blk_begin = groups;
    groups += (args.seg[i].N + kWaves * H - 1) / (kWaves * H);
  }
  // batch rows per launch column: each weight byte is read ceil(M / MC) times
  if (args.M >= 5) return launch_mc<QT, 8>(args, groups, H, s);
  if (args.M >= 3) return launch_mc<QT, 4>(args, groups, H, s);
  if (args.M == 2) return launch_mc<QT, 2>(args, groups, H, s);
  return launch_mc<QT, 1>(args, groups, H, s);
}

}  // namespace

bool gemv_packed_fits(int qtype, int K) {
  if (K <= 0) return false;
  switch (qtype) {
  case kTypeQ4_K:
  case kTypeQ6_K:
  case kTypeQ8_K: return K % 256 == 0;
  case kTypeQ8_0: return K % 32 == 0;
  default: return false;
  }
}

// count projections (1..3) of one quant type share the activations; fp16
// outputs [M][N[i]].
hipError_t launch_gemv_packed(int qtype, int count, const void *const *W, void *const *Y,
                              const int *N, const int8_t *X, const float *scales, int M, int K,
                              hipStream_t stream) {
  if (!gemv_packed_fits(qtype, K) || count < 1 || count > 3 || M < 0) return hipErrorInvalidValue;
  if (M == 0) return hipSuccess;
  PackedArgs args{};
  for (int i = 0; i < count; ++i)
    args.seg[i] = PackedSeg{static_cast<const uint8_t *>(W[i]), static_cast<uint16_t *>(Y[i]), N[i], 0};
  args.nseg = count;
  args.X = X;
  args.scales = scales;
  args.M = M;
  args.K = K;
  switch (qtype) {
  case kTypeQ4_K: return launch_qt<kTypeQ4_K>(args, stream);
  case kTypeQ6_K: return launch_qt<kTypeQ6_K>(args, stream);
  case kTypeQ8_0: return launch_qt<kTypeQ8_0>(args, stream);
  default: return launch_qt<kTypeQ8_K>(args, stream);
  }
}

}  // namespace ifx
