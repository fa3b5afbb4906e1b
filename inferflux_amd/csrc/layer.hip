// layer.hip -- the post-attention half of a decode layer at M = 1 in two
// launches instead of three: O accumulated into the fp32 residual (the GEMV
// with the fused Q8_1 quantizer, gemv.hip), then ONE launch for RMSNorm +
// Q8_1 of the residual, the gate/up GEMV with SiLU(gate) * up and its Q8_1
// blocks, and the down projection accumulated into the residual.
//
// Replaces the launch sequence of the reference's decode step
// (runtime/backends/cuda/native/transformer_forward.cu:726-817:
// GemvQ8_1AccumF32 for O, FusedRmsNormQuantizeQ8_1, the fused gate/up/SiLU
// GEMV with its Q8_1 epilogue, GemvQ8_1AccumF32 for down), which at M = 1 is
// bound by per-launch ramp and drain rather than by its 46 MB of weights.
//
// The FFN launch runs one workgroup of 16 waves per CU, all resident at
// once, in two phases separated by one grid barrier (a two-level arrival
// counter and a generation word in the caller's workspace, bounded waits):
//   start  waves 0-3 load the residual and norm weight and RMSNorm + Q8_1 it
//          into LDS; then every wave requests its gate or up rows of this
//          workgroup's equal share of the outputs (43 of 11008 at the 3B
//          shape, three rows per half-wave) into registers;
//   gate/up  row sums; waves 4-15 then request the workgroup's down rows (4
//          row pairs x 3 waves per pair) into registers, which stream while
//          h = silu(g) * u is written per output in fp32 to the workspace,
//          in 8 copies (one per group of workgroups: 256 workgroups reading
//          one copy queue on a few memory channels), and the barrier runs;
//   --- barrier (all of h is written) ---
//   down   each workgroup quantizes its group's copy of h to Q8_1 in LDS
//          (the standalone producer's blocks); waves 4-15 finish the rows
//          whose weights they hold: residual += down . Q8_1(h).
// Every row sum uses the lane-to-slice mapping and reduction order of the
// standalone kernel it replaces (k_gemv_swiglu_wide with the fused RMSNorm
// for gate/up, k_gemv with three waves per row pair for down), and h and its
// Q8_1 blocks use the producers' arithmetic, so the residual it leaves is
// bitwise the residual of the launch chain.
#include "ifx_slices.h"

namespace ifx {

struct FfnArgs {
  const uint8_t *Wg, *Wu, *Wd;
  float *resid;            // [hidden] fp32, updated in place
  const uint16_t *norm_w;  // [hidden] fp16: FFN RMSNorm weight
  float eps;
  float *hf;               // workspace: 8 copies of h, [ffn] fp32 each
  int64_t hf_copy;         // floats from one copy to the next
  uint32_t *ctl;           // workspace: arrival count, generation, error
  int hidden, ffn;
  int gd;                  // waves per down row pair (ceil(ffn / 64 / 64))
};

// Workspace layout (uint32 words): [0] top arrival count, [1] generation,
// [2] failure flag, bytes 16..23 an int64 wait limit in realtime-clock ticks
// (100 MHz; 0 = 1 s), [64 + 32 j] the arrival count of workgroup group j
// (j = blockIdx % 8, one 128-byte line each); from byte kFfnCtlBytes, 8
// copies of h in fp32 (copy j read by group j), each padded to a multiple of
// 256 bytes.  The control block is zero before the first call.
constexpr long long kDefaultSpinTicks = 100000000;
constexpr int kFfnCtlBytes = 2048;
constexpr int kFfnGroups = 8;

constexpr int kFfnMaxK = 2048;     // hidden: half-wave rows (<= 32 wide slices)
constexpr int kFfnMaxFfn = 16384;  // ffn: one wide down slice per lane (3 waves of 64)
constexpr int kFfnR = 3;           // gate (up) rows per half-wave: 16 half-waves x 3 = 48
constexpr int kFfnGuRows = 16 * kFfnR;  // outputs per workgroup at most
constexpr int kFfnDownWaves = 12;  // waves 4-15 hold the down rows


// Grid barrier over all workgroups of the launch (all resident: one per CU),
// in two halves so a workgroup can issue loads between arriving and
// waiting.  Data that crosses workgroups is written with device-coherent
// stores, and every wave that wrote some has waited for its stores
// (wait_own_memory) before arriving, and is read back with device-coherent
// loads, so no cache write-back or invalidation is needed.  Arrival is
// two-level (measured on MI355X: about 2 us per barrier against 4 us for one
// counter that all 256 workgroups hit): thread 0 adds to its group's counter
// (blockIdx % 8), the last of a group adds to the top counter, and the last
// group resets the counters and advances the generation; the others poll
// the generation, at most `limit` ticks, then record a failure in ctl[2] and
// go on (every wave still reaches the end of the kernel).
struct GridBarrier {
  uint32_t *ctl;
  uint32_t gen;
  bool last;

  __device__ __forceinline__ void arrive(uint32_t nwg) {
    __syncthreads();
    if (threadIdx.x == 0) {
      gen = __hip_atomic_load(ctl + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      const uint32_t grp = blockIdx.x % kFfnGroups;
      const uint32_t ngrp = nwg < kFfnGroups ? nwg : kFfnGroups;
      const uint32_t per = (nwg - grp + kFfnGroups - 1) / kFfnGroups;  // workgroups in the group
      uint32_t *gc = ctl + 64 + 32 * grp;
      last = false;
      if (__hip_atomic_fetch_add(gc, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == per - 1) {
        __hip_atomic_store(gc, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        last = __hip_atomic_fetch_add(ctl, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
               ngrp - 1;
      }
      if (last) {
        __hip_atomic_store(ctl, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(ctl + 1, gen + 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
  }

  __device__ __forceinline__ void wait(long long limit) {
    if (threadIdx.x == 0 && !last) {
      const long long t0 = wall_clock64();
      while (__hip_atomic_load(ctl + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == gen) {
        if (wall_clock64() - t0 > limit) {
          __hip_atomic_store(ctl + 2, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          break;
        }
        __builtin_amdgcn_s_sleep(1);
      }
    }
    __syncthreads();
  }
};

// Phase timestamps for tuning builds (-DIFX_FFN_TRACE): thread 0 of each
// workgroup writes the realtime clock at each phase boundary to 8 int64 slots
// per workgroup after the h blocks in the workspace.
#ifdef IFX_FFN_TRACE
#define IFX_FFN_STAMP(i)                                                              \
  do {                                                                              \
    if (threadIdx.x == 0)                                                           \
      reinterpret_cast<long long *>(args.hf + 8 * args.hf_copy) \
          [blockIdx.x * 8 + (i)] = wall_clock64();                                  \
  } while (0)
#else
#define IFX_FFN_STAMP(i) \
  do {                   \
  } while (0)
#endif

__global__ __launch_bounds__(1024) void k_decode_ffn(const FfnArgs args) {
  __shared__ __attribute__((aligned(16))) uint8_t a_lds[(kFfnMaxK / 32) * kQ8_1Bytes];
  __shared__ __attribute__((aligned(16))) float r_lds[kFfnMaxK];  // the residual
  __shared__ __attribute__((aligned(16))) uint8_t h_lds[(kFfnMaxFfn / 32) * kQ8_1Bytes];  // Q8_1 of h
  __shared__ float npart[4];
  __shared__ float gu[2][kFfnGuRows];  // [gate/up][output of this workgroup]
  __shared__ float red[kFfnDownWaves * 2];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int half = lane >> 5, lt = lane & 31;
  const int nwg = gridDim.x, wg = blockIdx.x;
  const int hidden = args.hidden, ffn = args.ffn;
  long long spin = *reinterpret_cast<const long long *>(args.ctl + 4);
  if (spin <= 0) spin = kDefaultSpinTicks;
  IFX_FFN_STAMP(0);

  // Loads are issued unconditionally: a wave or lane with nothing to load
  // reads through an empty buffer range or at an offset past it, which
  // returns zeros without touching memory.  With no branches around them the
  // compiler waits for exactly the loads each step needs (a wave's loads
  // complete in issue order).
  constexpr uint32_t kNone = 0xFFFFF000u;  // an offset past every range here

  // ------------------------------------- the residual and norm weight
  // (waves 0-3).  They arrive before anything else is requested: a load
  // queued behind the 44 MB weight stream would wait for most of it.  The
  // residual is also kept in LDS for the down projection's accumulate.
  f32x4 xr[2];
  u32x2 wr[2];
  {
    const rsrc_t Xr = make_rsrc(args.resid, wave < 4 ? hidden * 4u : 0u);
    const rsrc_t Nr = make_rsrc(args.norm_w, wave < 4 ? hidden * 2u : 0u);
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const uint32_t i = 4 * threadIdx.x + 1024 * j;
      xr[j] = bload<f32x4>(Xr, i * 4, 0);
      wr[j] = bload<u32x2>(Nr, i * 2, 0);
    }
  }
  if (wave < 4) {
#pragma unroll
    for (int j = 0; j < 2; ++j)
      if (4 * static_cast<int>(threadIdx.x) + 1024 * j < hidden)
        *reinterpret_cast<f32x4 *>(r_lds + 4 * threadIdx.x + 1024 * j) = xr[j];
    rmsnorm_row_partial<2>(xr, hidden, npart, threadIdx.x);
  }
  __syncthreads();

  // -------------------------------------- RMSNorm + Q8_1 of the residual
  // (k_gemv_swiglu_wide's producer prologue)
  const uint32_t ag_row = static_cast<uint32_t>(hidden >> 5) * kQ8_1Bytes;
  if (wave < 4) rmsnorm_row_apply<2>(xr, wr, a_lds, hidden, args.eps, npart, threadIdx.x);
  __syncthreads();
  IFX_FFN_STAMP(1);

  // ---------------------------------------------- weights, into registers
  // Gate/up: this workgroup's outputs [o0, o0 + ocnt) (an equal share of
  // ffn); waves 0-7 take the gate rows, 8-15 the up rows, kFfnR rows per
  // half-wave; requested now (a workgroup barrier waits for every wave to
  // finish issuing its loads, so the stream starts after the producer's
  // barriers).  Down: row pair dgrp (rows 2 dgrp, 2 dgrp + 1) is held by
  // waves 4 + gd j .. 4 + gd j + gd - 1; wave dgw of the pair takes wide
  // slice dgw * 64 + lane (one slice per lane: 64 gd >= ffn / 64).
  const int oper = (ffn + nwg - 1) / nwg;
  const int o0 = wg * oper, ocnt = max(0, min(oper, ffn - o0));
  const bool is_up = wave >= 8;
  const int hw = (wave & 7) * 2 + half;  // half-wave index among the 16 of gate or up
  const uint32_t g_row = static_cast<uint32_t>(row_bytes(kTypeQ4_K, hidden));
  const int nslice_g = hidden >> 6;
  const rsrc_t Wgr = make_rsrc(is_up ? args.Wu : args.Wg, g_row * static_cast<uint32_t>(ffn));
  const uint32_t gsoff[kFfnR] = {};
  uint32_t gvoff[kFfnR];
#pragma unroll
  for (int r = 0; r < kFfnR; ++r) {
    const int o = hw * kFfnR + r;  // output within the workgroup's range
    gvoff[r] = (o < ocnt && lt < nslice_g) ? static_cast<uint32_t>(o0 + o) * g_row : kNone;
  }
  Q4Wide<kFfnR> gwt;
  q4k_wide_load<kFfnR>(gwt, Wgr, gvoff, gsoff, lt < nslice_g ? lt : 0);

  const int gd = args.gd;
  const int dpairs = (hidden + 1) >> 1;
  const int dpw = (dpairs + nwg - 1) / nwg;  // row pairs per workgroup
  const int dloc = (wave - 4) / gd, dgw = (wave - 4) % gd;
  const int dgrp = wg * dpw + dloc;
  const bool dwave = wave >= 4 && dloc < dpw && dgrp < dpairs;
  const int nslice_d = ffn >> 6;
  const int ds = dgw * 64 + lane;
  const bool dlane = dwave && ds < nslice_d;
  const uint32_t d_row = static_cast<uint32_t>(row_bytes(kTypeQ6_K, ffn));
  const rsrc_t Wdr = make_rsrc(args.Wd, dwave ? d_row * static_cast<uint32_t>(hidden) : 0u);
  uint32_t dvoff[2];
  const uint32_t dsoff[2] = {0u, 0u};
#pragma unroll
  for (int r = 0; r < 2; ++r)
    dvoff[r] = dlane ? static_cast<uint32_t>(min(2 * dgrp + r, hidden - 1)) * d_row : kNone;
  Q6Wide<2> dwt;  // requested once this wave's gate/up rows are summed

  // ------------------------------------------- gate/up row sums, then h
  {
    const ALds gas{a_lds, ag_row};
    float acc[kFfnR][1] = {};
    for (int s = lt; s < nslice_g; s += 32) {
      if (s != lt) q4k_wide_load<kFfnR>(gwt, Wgr, gvoff, gsoff, s);
      q4k_wide_compute<1, kFfnR>(gwt, gas, 1, s, acc);
    }
#pragma unroll
    for (int r = 0; r < kFfnR; ++r) {
      const float v = halfwave_sum_to31(acc[r][0]);
      const int o = hw * kFfnR + r;
      if (lt == 31 && o < kFfnGuRows) gu[is_up][o] = v;
    }
  }
  // the down weights: requested after the gate/up sums (a wave's loads
  // complete in order, so earlier they would hold up its gate/up data, and
  // a wave cannot compute while its load issue is stalled on a full queue)
  q6k_wide_load<2>(dwt, Wdr, dvoff, dsoff, dlane ? ds : 0);
  __syncthreads();
  // h = silu(g) * u of each output (the SiLU producer's arithmetic), in fp32,
  // to the 8 copies (one per group of workgroups: 256 workgroups reading one
  // copy would queue on a few memory channels); device-coherent stores
  for (int t = threadIdx.x; t < 8 * ocnt; t += 1024) {
    const int o = t % ocnt, c = t / ocnt;
    const float g = gu[0][o], u = gu[1][o];
    const float h = silu_mul1(g, u);
    __hip_atomic_store(args.hf + c * args.hf_copy + o0 + o, h, __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
  }
  if (wave <= (8 * kFfnGuRows - 1) / 64) wait_own_memory();  // h is stored before arriving
  IFX_FFN_STAMP(2);
  GridBarrier gb{args.ctl, 0u, false};
  gb.arrive(nwg);
  gb.wait(spin);
  IFX_FFN_STAMP(3);

  // --------------------- Q8_1 of h into LDS, from this workgroup's copy
  // (device-coherent loads: other workgroups wrote it; the standalone
  // producer's blocks, 8 lanes per block of 32)
  {
    const float *hsrc = args.hf + (wg % kFfnGroups) * args.hf_copy;
    const rsrc_t Hr = make_rsrc(hsrc, ffn * 4u);
    for (int t = threadIdx.x; t < (ffn >> 5) * 8; t += 1024) {
      const f32x4 v = __builtin_bit_cast(
          f32x4, __builtin_amdgcn_raw_buffer_load_b128(Hr, 16 * t, 0, 0x10 /* sc1 */));
      quantize4_store(v.x, v.y, v.z, v.w, h_lds + (t >> 3) * kQ8_1Bytes, t & 7);
    }
  }
  __syncthreads();

  // ------------------------------------------ down: residual += down . Q8_1(h)
  const uint32_t ad_row = static_cast<uint32_t>(ffn >> 5) * kQ8_1Bytes;
  float dacc[2][1] = {{0.0f}, {0.0f}};
  if (dlane) q6k_wide_compute<1, 2>(dwt, ALds{h_lds, ad_row}, 1, ds, dacc);
  float v[2];
#pragma unroll
  for (int r = 0; r < 2; ++r) v[r] = wave_sum_to63(dacc[r][0]);
  if (wave >= 4 && lane == 63) {
    red[(wave - 4) * 2] = v[0];
    red[(wave - 4) * 2 + 1] = v[1];
  }
  __syncthreads();
  if (dwave && dgw == 0 && lane == 63) {
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      float t = 0.0f;
      for (int w = 0; w < gd; ++w) t += red[(dloc * gd + w) * 2 + r];
      const int row = 2 * dgrp + r;
      if (row < hidden) args.resid[row] = t + r_lds[row];
    }
  }
  IFX_FFN_STAMP(4);
}

namespace {
constexpr int kMaxDev = 64;
int g_ncu[kMaxDev];
}  // namespace

// Compute units of the current device (the grid: one workgroup per CU).
static int device_cus() {
  if (dry_run()) return 256;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDev) return 0;
  if (!g_ncu[dev]) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
    g_ncu[dev] = n;
  }
  return g_ncu[dev];
}

// Whether the FFN kernel covers the shape on this device: half-wave rows for
// gate/up (hidden <= 2048), at most one wide down slice per lane (ffn <=
// 16384) and the down rows of a workgroup within its 12 holding waves.
bool decode_ffn_fits(int hidden, int ffn) {
  if (hidden <= 0 || ffn <= 0 || hidden % 256 || ffn % 256) return false;
  if (hidden > kFfnMaxK || ffn > kFfnMaxFfn) return false;  // (every tensor < 64 MB: below kNone)
  const int ncu = device_cus();
  if (ncu <= 0) return false;
  const int gd = (ffn / 64 + 63) / 64;
  const int dpw = ((hidden + 1) / 2 + ncu - 1) / ncu;
  return dpw * gd <= kFfnDownWaves && (ffn + ncu - 1) / ncu <= kFfnGuRows;
}

hipError_t launch_gemv_rmsnorm(int count, const void *const *W, void *const *Y, const int *N,
                               const void *x, bool x_f16, const uint16_t *norm_w, float eps,
                               bool f16, int M, int K, int mode, hipStream_t stream);

// O accumulated into the residual (the GEMV with the fused quantizer; none
// when Wo is NULL), then the FFN kernel.
hipError_t launch_decode_ffn(const void *Wo, const void *attn, bool attn_f16, float *resid,
                             const uint16_t *norm_w, float eps, const void *Wg, const void *Wu,
                             const void *Wd, void *workspace, int q_dim, int hidden, int ffn,
                             hipStream_t s) {
  if (!decode_ffn_fits(hidden, ffn)) return hipErrorInvalidValue;
  if (Wo) {  // NULL: the residual already holds the attention block's output
    void *y = resid;
    const hipError_t e = launch_gemv_rmsnorm(1, &Wo, &y, &hidden, attn, attn_f16, nullptr, 0.0f,
                                             false, 1, q_dim, 1 /* accumulate */, s);
    if (e != hipSuccess) return e;
  }
  FfnArgs a;
  a.Wg = static_cast<const uint8_t *>(Wg);
  a.Wu = static_cast<const uint8_t *>(Wu);
  a.Wd = static_cast<const uint8_t *>(Wd);
  a.resid = resid;
  a.norm_w = norm_w;
  a.eps = eps;
  a.ctl = static_cast<uint32_t *>(workspace);
  a.hf = reinterpret_cast<float *>(static_cast<uint8_t *>(workspace) + kFfnCtlBytes);
  a.hf_copy = (static_cast<int64_t>(ffn) + 63) / 64 * 64;
  a.hidden = hidden;
  a.ffn = ffn;
  a.gd = (ffn / 64 + 63) / 64;
  const dim3 grid(static_cast<unsigned>(device_cus()));
  IFX_LAUNCH0(k_decode_ffn, grid, dim3(1024), 0, s, a);
  return last_error();
}

}  // namespace ifx
