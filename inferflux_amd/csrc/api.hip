// api.hip -- the C ABI (include/ifx_qgemm.h): argument validation and
// dispatch by quant type and batch size onto the gfx950 kernels.
//
// Validation mirrors FusedQuantGemm::GemvQ8_1
// (runtime/backends/cuda/native/fused_quant_gemm.cu:2085-2117): a NULL
// pointer, an unsupported type or a bad geometry is "not handled" (a positive
// status, the reference's `false`) and launches nothing.  Unlike the
// reference, launch errors are checked (hipGetLastError after each launch)
// and returned as a negative status.
#include "../../include/ifx_qgemm.h"
#include "ifx_q8_1.h"

#include <stdlib.h>

#include <algorithm>

#include <string>

namespace ifx {
hipError_t launch_quantize_q8_1(const void *x, bool f16, void *out, int64_t M, int64_t K,
                                hipStream_t stream);
hipError_t launch_rmsnorm_quantize_q8_1(const void *x, bool f16, const uint16_t *w, void *out,
                                        int M, int K, float eps, hipStream_t stream);
hipError_t launch_silu_mul_quantize_q8_1(const void *g, const void *u, bool f16, void *out,
                                         int64_t M, int64_t K, hipStream_t stream);
hipError_t launch_dequantize(int qtype, const void *W, void *out, bool f16, int64_t n_elems,
                             hipStream_t stream);
hipError_t launch_gemv(int qtype, const void *W, const void *A, void *Y, const void *bias,
                       bool f16, int M, int N, int K, int mode, hipStream_t stream);
hipError_t launch_gemv_grouped(int qtype, int count, const void *const *W, void *const *Y,
                               const int *N, const void *A, bool f16, int M, int K, int mode,
                               hipStream_t stream);
hipError_t launch_gemv_swiglu(int qtype, const void *Wg, const void *Wu, const void *A, void *H,
                              bool f16h, void *Q, int M, int N, int K, hipStream_t stream);
hipError_t launch_gemv_swiglu_rmsnorm(const void *Wg, const void *Wu, const void *x, bool x_f16,
                                      const uint16_t *norm_w, float eps, void *H, bool f16h,
                                      void *Q, int M, int N, int K, hipStream_t stream);
hipError_t launch_mmvq(int qtype, int count, const void *const *W, void *const *Y,
                       const int *N, const void *bias, const void *A, bool f16, int M, int K,
                       int mode, hipStream_t stream);
hipError_t launch_mmq_skinny(int qtype, int count, const void *const *W, void *const *Y,
                             const int *N, const void *bias, const void *A, bool f16, int M,
                             int K, int mode, hipStream_t stream);
hipError_t launch_gemm_mfma(int qtype, const void *W, const void *A, void *Y, const void *bias,
                            bool f16, int M, int N, int K, int mode, hipStream_t stream);
bool gemv_lds_fits(int qtype, int M, int K);
hipError_t launch_gemv_lds(int count, const void *const *W, void *const *Y, const int *N,
                           const void *bias, const void *A, bool f16, int M, int K, int mode,
                           hipStream_t stream);
bool gemm_f16_fits(int qtype, int K);
int64_t gemm_f16_workspace_bytes(int M, int K);
hipError_t launch_gemm_f16(int qtype, const void *W, const void *A, void *A16, void *Y, const void *bias,
                           bool f16, int M, int N, int K, int mode, int splits_req,
                           hipStream_t stream, float *slots = nullptr);
int64_t gemm_f16_slot_bytes(bool f16, int M, int N, int K);
hipError_t launch_gemv_rmsnorm(int count, const void *const *W, void *const *Y, const int *N,
                               const void *x, bool x_f16, const uint16_t *norm_w, float eps,
                               bool f16, int M, int K, int mode, hipStream_t stream);
bool gemv_dq_fits(int qtype, int M, int K);
bool gemv_dq_fits_f16(int M, int K);
bool gemv_dq_f16_unsplit(int count, const int *N, int M, int K);
hipError_t launch_gemv_dq(int qtype, int count, const void *const *W, void *const *Y,
                          const int *N, const void *bias, const void *A, bool f16, int M, int K,
                          int mode, int splits_req, hipStream_t stream, void *ws = nullptr);
int64_t gemv_dq_workspace_bytes(int count, const int *N, bool f16, int M, int K);
hipError_t scratch_address(void **out);
hipError_t launch_repack(int qtype, const void *W, void *out, int64_t n_rows, int K,
                         hipStream_t stream);
hipError_t launch_repack_tiled(int qtype, const void *W, void *out, int64_t n_rows, int K,
                               hipStream_t stream);
bool gemv_slot_fits(int qtype, int M, int K);
int gemv_dq_swiglu_splits(int M, int N, int K);
hipError_t launch_gemv_dq_swiglu(int qtype, const void *Wg, const void *Wu, const void *A,
                                 void *H, bool h_f16, void *Q, int M, int N, int K, void *ws,
                                 hipStream_t stream);
int64_t gemv_dq_workspace_bytes(int count, const int *N, bool f16, int M, int K);
hipError_t launch_gemv_slot_swiglu(int qtype, const void *Wg, const void *Wu, const void *A,
                                   void *H, bool f16h, void *Q, int M, int N, int K,
                                   hipStream_t stream);
hipError_t launch_gemv_slot(int qtype, int count, const void *const *W, void *const *Y,
                            const int *N, const void *bias, const void *A, bool f16, int M, int K,
                            int mode, hipStream_t stream, void *ws = nullptr);
int64_t gemv_slot_workspace_bytes(int count, const int *N, bool f16, int M, int K);
hipError_t launch_quantize_rows_sym(const void *a, const void *b, int dtype, int8_t *codes,
                                    float *scales, int M, int K, hipStream_t stream);
bool gemv_packed_fits(int qtype, int K);
hipError_t launch_gemv_packed(int qtype, int count, const void *const *W, void *const *Y,
                              const int *N, const int8_t *X, const float *scales, int M, int K,
                              hipStream_t stream);
}  // namespace ifx

// ---------------------------------------------------------------- launch log
namespace ifx {
namespace {
struct LaunchLog {
  bool open = false, dry = false;
  std::string text;
};
thread_local LaunchLog g_log;
}  // namespace

bool note_launch(const char *kernel, std::initializer_list<int> targs) {
  if (g_log.open) {
    if (!g_log.text.empty()) g_log.text += ';';
    g_log.text += kernel;
    if (targs.size()) {
      g_log.text += '<';
      bool first = true;
      for (int v : targs) {
        if (!first) g_log.text += ',';
        g_log.text += std::to_string(v);
        first = false;
      }
      g_log.text += '>';
    }
  }
  return !g_log.dry;
}
bool dry_run() { return g_log.dry; }
hipError_t last_error() { return g_log.dry ? hipSuccess : hipGetLastError(); }
hipError_t peek_error() { return g_log.dry ? hipSuccess : hipPeekAtLastError(); }
}  // namespace ifx

namespace {

// Batch-size dispatch (the reference's MMVQ / MMQ / cuBLAS split,
// fused_quant_gemm.cu:1697-1747, re-derived for gfx950):
//   M <= 2       v_dot4 GEMV        (gemv.hip)
//   3 <= M <= 32 skinny int8 MFMA   (mmq_skinny.hip), K % 256 == 0
//   M > 32       tiled int8 MFMA    (gemm_mfma.hip)
//   M >= 33 (Q6_K), 96 (Q4_K), 128 (Q8_0): fp16 MFMA with in-kernel dequant
//                (gemm_f16.hip), the reference's FP16 prefill arithmetic
constexpr int kMaxGemvMDefault = 2;
constexpr int kMaxSkinnyM = 32;
// Prefill kernel for M > 32: the fp16 GEMM from min_f16_gemm_m(qtype) rows
// on, else the int8 MFMA GEMM.  Measured at the 32B shapes (graph-replayed,
// us for fp16 / int8): Q6_K 5120 x 27648 M = 48: 111 / 438, M = 128: 118 /
// 438 (the int8 kernel's per-block rescale of 16-value Q6_K groups); Q4_K
// 27648 x 5120 M = 48: 104 / 63, M = 64: 98 / 64, M = 96: 99 / 105, M = 128:
// 102 / 104.  Q8_0 is unmeasured and keeps 128 (a 256-row tile is mostly
// padding below that).  IFX_PREFILL=int8|f16 forces one (tuning; read once).
int min_f16_gemm_m(int qtype) {
  return qtype == IFX_TYPE_Q6_K ? kMaxSkinnyM + 1 : qtype == IFX_TYPE_Q4_K ? 96 : 128;
}

bool use_f16_gemm(int qtype, int M, int K) {
  static const int v = [] {
    const char *e = ifx::tuning_env("IFX_PREFILL");
    return e ? (e[0] == 'i' ? 1 : e[0] == 'f' ? 2 : 0) : 0;
  }();
  if (!ifx::gemm_f16_fits(qtype, K) || v == 1) return false;
  return v == 2 || M >= min_f16_gemm_m(qtype);
}
// Q5_K and Q8_K run on the v_dot4 GEMV only, for M <= 64: the reference's
// Q8_K dispatch stops at 64 (fused_quant_gemm.cu:1740-1747) and it has no
// fused Q5_K kernel at all (dequantize + cuBLAS); larger M is "not handled".
constexpr int kMaxGemvOnlyM = 64;

// Largest M the v_dot4 GEMV takes; IFX_GEMV_MAX_M in 0..8 overrides it
// (tuning; read once).
int max_gemv_m() {
  static const int v = [] {
    const char *e = ifx::tuning_env("IFX_GEMV_MAX_M");
    const int n = e ? atoi(e) : 0;
    return (n >= 0 && n <= 8 && e) ? n : kMaxGemvMDefault;
  }();
  return v;
}

// Decode-batch kernel for 3 <= M <= 32 (measured on MI355X): the MFMA GEMV
// with a per-workgroup K split (mmvq.hip) up to M = 16; above it the
// workgroup-shared activation tile of mmq_skinny.hip reads fewer bytes per
// weight byte.  IFX_DECODE=skinny|mmvq forces one (tuning; read once).
bool use_skinny(int M) {
  static const int v = [] {
    const char *e = ifx::tuning_env("IFX_DECODE");
    return e ? (e[0] == 's' ? 1 : e[0] == 'm' ? 2 : 0) : 0;
  }();
  return v == 1 || (v == 0 && M > 16);
}

// Q4_K decode batches where the GEMV with activations in LDS
// (gemv_lds.hip) beats the MFMA kernel, measured on MI355X with cold
// weights: M = 3 (K <= 5120), and M = 4 on wide launches (K <= 2048, at
// least 16384 rows).  Its VALU work grows with M, so M >= 5 stays on MFMA.
// IFX_LDS=0|1 forces it off / on for every shape it fits (tuning; read once).
bool use_lds(int qtype, int M, int K, int n_total) {
  static const int v = [] {
    const char *e = ifx::tuning_env("IFX_LDS");
    return e ? (e[0] == '1' ? 1 : e[0] == '2' ? 2 : 0) : -1;
  }();
  if (!ifx::gemv_lds_fits(qtype, M, K) || v == 0) return false;
  if (v == 1) return true;
  return M == 3 || (M == 4 && K <= 2048 && n_total >= 16384);
}

// Q4_K / Q6_K decode batches on the slot-packed MFMA GEMV (gemv_slot.hip),
// measured on MI355X with cold weights against the LDS-staged MFMA kernel:
// 5 <= M <= 8 on launches of at least 8192 rows (gate/up, LM head), and
// 3 <= M <= 8 on long-K launches with fp32 outputs (K >= 8192: the down
// projection, 2048 x 11008 Q6_K at M = 3 / 4: 12.7 / 12.9 us against 13.9 /
// 14.5 on mmvq.hip), which it splits over several workgroups, and
// 4 <= M <= 8 on launches of at most 24 super-blocks per row (Q/K/V and O,
// 8 waves, no split: 3B O at M = 4 / 8 4.8 / 5.0 us against 5.1 / 5.2 on
// mmvq.hip; 14B O 5120 x 5120 at M = 8 7.2 against 8.9).  IFX_SLOT=0|1
// forces it off / on for every M it fits (1..8; tuning; read once).
bool use_slot(int qtype, int M, int K, int n_total, bool f16) {
  static const int v = [] {
    const char *e = ifx::tuning_env("IFX_SLOT");
    return e ? (e[0] == '1' ? 1 : e[0] == '2' ? 2 : 0) : -1;
  }();
  if (!ifx::gemv_slot_fits(qtype, M, K) || v == 0) return false;
  if (v == 1) return true;
  return (M >= 5 && n_total >= 8192) || (M >= 3 && K >= 8192 && !f16) || (M >= 4 && K <= 6144);
}

// Decode batches 17 <= M <= 32 on the fp16-dequant MFMA GEMV (gemv_dq.hip),
// measured on MI355X with cold weights against mmq_skinny.hip: 14B gate
// 13824 x 5120 Q4_K M = 32: 25.6 us (33.8); 14B down 5120 x 13824 Q6_K:
// 30.3 us (53.3); 3B gate 11008 x 2048: 12.5 us (15.8).  Its VALU work per
// weight does not grow with M; below M = 17 the integer kernels are faster.
// IFX_DQ=0|1 forces it off / on for every M it fits (1..32; tuning; read
// once); IFX_DQ=0 also keeps tiled launches up to M = 16 on the slot kernel.
int dq_env() {
  static const int v = [] {
    const char *e = ifx::tuning_env("IFX_DQ");
    return e ? (e[0] == '1' ? 1 : e[0] == '2' ? 2 : 0) : -1;
  }();
  return v;
}
bool use_dq(int qtype, int M, int K, bool f16) {
  const int v = dq_env();
  if (!ifx::gemv_dq_fits(qtype, M, K) || (f16 && !ifx::gemv_dq_fits_f16(M, K)) || v == 0)
    return false;
  return v == 1 || M > 16;
}

int status_of(hipError_t e) { return e == hipSuccess ? IFX_OK : -static_cast<int>(e); }

bool gemv_only(int t) { return t == IFX_TYPE_Q5_K || t == IFX_TYPE_Q8_K; }

// the row-split layouts of ifx_repack: the v_dot4 GEMV at M <= 2 only
bool row_split(int t) { return t == IFX_TYPE_Q8_0_R || t == IFX_TYPE_Q6_K_R; }
constexpr int kMaxRowSplitM = 2;
// the tiled layouts of ifx_repack_tiled: the MFMA batch GEMVs, M <= 32
bool tiled(int t) { return t == IFX_TYPE_Q4_K_T || t == IFX_TYPE_Q6_K_T || t == IFX_TYPE_Q8_0_T; }
constexpr int kMaxTiledM = 32;
constexpr int kMaxSlotM = 8;
// a layout of this library, served by some entry points only
bool repacked(int t) { return row_split(t) || tiled(t); }

bool is_weight_type(int t) {
  return t == IFX_TYPE_Q4_K || t == IFX_TYPE_Q6_K || t == IFX_TYPE_Q8_0 || gemv_only(t) ||
         repacked(t);
}

// Bytes of an N x K weight tensor (0 for an unknown type); tiled tensors
// hold whole groups of 32 rows.
uint64_t weight_bytes(int t, int N, int K) {
  if (!ifx_block_elems(t)) return 0;
  const uint64_t rows = tiled(t) ? (static_cast<uint64_t>(N) + 31) / 32 * 32 : N;
  return rows * ifx::row_bytes(t, K);
}

// Kernels address W and A with 32-bit byte offsets (buffer loads) and read
// zeros at ifx::kOobOffset, past every accepted tensor.
bool buffers_fit(int quant_type, int M, int N, int K) {
  if (N > (1 << 30) || M > (1 << 24) || K > (1 << 24)) return false;
  const uint64_t w_bytes = weight_bytes(quant_type, N, K);
  const uint64_t a_bytes = static_cast<uint64_t>(M) * (K / 32) * 36;
  return w_bytes < ifx::kMaxBufferBytes && a_bytes < ifx::kMaxBufferBytes;
}

int check_gemm_args(int quant_type, const void *W, const void *A, void *Y, int out_dtype,
                    int mode, const void *bias, int M, int N, int K) {
  if (!W || !A || !Y) return IFX_NULL_POINTER;
  if (!is_weight_type(quant_type)) return IFX_UNSUPPORTED_TYPE;
  if (out_dtype != IFX_OUT_F32 && out_dtype != IFX_OUT_F16) return IFX_BAD_GEOMETRY;
  if (mode != IFX_STORE && mode != IFX_ACCUM && mode != IFX_BIAS) return IFX_BAD_GEOMETRY;
  if (mode == IFX_BIAS && !bias) return IFX_NULL_POINTER;
  if (M <= 0 || N <= 0 || K <= 0) return IFX_BAD_GEOMETRY;
  if (K % ifx_block_elems(quant_type) != 0) return IFX_BAD_GEOMETRY;
  if (gemv_only(quant_type) && M > kMaxGemvOnlyM) return IFX_BAD_GEOMETRY;
  if (row_split(quant_type) && M > kMaxRowSplitM) return IFX_BAD_GEOMETRY;
  if (tiled(quant_type) && M > kMaxTiledM) return IFX_BAD_GEOMETRY;
  if (!buffers_fit(quant_type, M, N, K)) return IFX_BAD_GEOMETRY;
  return IFX_OK;
}

// Kernel route of ifx_qgemv (grouped = false) and ifx_qgemv_grouped
// (grouped = true) for valid arguments; n_total = sum of the projections' N.
// atomic_accum: a plain entry (no ordered reduction asked for) accumulating
// into fp32 outputs.  Such Q4_K / Q6_K launches at 9 <= M <= 16 take the
// fp16-dequant GEMV's atomic K split, which needs no zero fill in that mode
// (measured on MI355X, 14B O / down at M = 16: 7.2 / 18.2 us against 10.3 /
// 20.5 tiled on the slot GEMV, 7.6 / 27.1 against 10.3 / 31.2 raw on MMVQ;
// 3B O 4.5 against 6.4) when they have 2048 rows or more; the store
// launches and the ordered entries keep the integer kernels (the zero fill,
// or the split's ordered reduction, costs more than it gains), and so do
// narrow launches (integer-exact sums: a row of few outputs is no norm to
// hide the fp16 weight rounding behind).
enum class Route { F16Gemm, Gemv, Lds, Slot, Dq, Skinny, Mmvq, Mfma, PerProjection };
Route route(int qt, int M, int K, int n_total, bool f16, bool grouped, bool atomic_accum = false) {
  static const int acc_min_m = [] {  // IFX_ACCUM_DQ_MIN_M (tuning; read once)
    const char *e = ifx::tuning_env("IFX_ACCUM_DQ_MIN_M");
    return e && atoi(e) > 0 ? atoi(e) : kMaxSlotM + 1;
  }();
  if (atomic_accum && !f16 && M >= acc_min_m && M <= 2 * kMaxSlotM && n_total >= 2048 &&
      dq_env() < 0 &&
      (qt == IFX_TYPE_Q4_K || qt == IFX_TYPE_Q6_K || qt == IFX_TYPE_Q4_K_T ||
       qt == IFX_TYPE_Q6_K_T) &&
      ifx::gemv_dq_fits(qt, M, K))
    return Route::Dq;
  if (tiled(qt)) {
    // measured on MI355X (14B / 3B shapes, cold weights): the slot-packed
    // GEMV (two 16-row slots above M = 8) up to M = 16, except wide Q4_K
    // launches from M = 9 (14B gate+up M = 12: 25.6 us on the fp16-dequant
    // GEMV against 29.5); the fp16-dequant GEMV above M = 16 (Q6_K down
    // 5120 x 13824 M = 16: 19.0 us on the slot GEMV, 20.9 on fp16-dequant)
    if (M <= kMaxSlotM) return Route::Slot;
    if (M <= 2 * kMaxSlotM && dq_env() != 2 &&
        (qt == IFX_TYPE_Q6_K_T || n_total < 8192 || dq_env() == 0))
      return Route::Slot;
    return Route::Dq;
  }
  if (!grouped && !gemv_only(qt) && M > kMaxSkinnyM && use_f16_gemm(qt, M, K)) return Route::F16Gemm;
  if (gemv_only(qt) || row_split(qt) || M <= max_gemv_m() || (M > kMaxSkinnyM && K % 256 != 0))
    return Route::Gemv;
  if (use_lds(qt, M, K, n_total)) return Route::Lds;
  if (use_slot(qt, M, K, n_total, f16)) return Route::Slot;
  if (use_dq(qt, M, K, f16)) return Route::Dq;
  if (M <= kMaxSkinnyM) return (use_skinny(M) && K % 256 == 0) ? Route::Skinny : Route::Mmvq;
  return grouped ? Route::PerProjection : Route::Mfma;
}

// The ordered-split workspace of a slot / dq launch: nullptr when there is
// none (atomics) or the launch does not split; rc = IFX_BAD_GEOMETRY when
// the caller's workspace is too small or not 256-byte aligned.
// ordered: an ordered entry (ifx_qgemv_ws / _grouped_ws), whose launches
// that split need the workspace (none given: IFX_BAD_GEOMETRY).
void *split_ws(Route r, void *ws, int64_t ws_bytes, int count, const int *N, bool f16,
               int M, int K, bool ordered, int &rc) {
  rc = IFX_OK;
  if (!ws && !ordered) return nullptr;
  const int64_t need = r == Route::Slot ? ifx::gemv_slot_workspace_bytes(count, N, f16, M, K)
                                        : ifx::gemv_dq_workspace_bytes(count, N, f16, M, K);
  if (need == 0) return nullptr;
  if (!ws || ws_bytes < need || reinterpret_cast<uintptr_t>(ws) % 256 != 0) rc = IFX_BAD_GEOMETRY;
  return ws;
}

int qgemv_impl(int quant_type, const void *W, const void *A_q8_1, void *Y, int out_dtype, int mode,
               const void *bias, int M, int N, int K, void *stream, void *ws, int64_t ws_bytes,
               bool ordered) {
  const int rc = check_gemm_args(quant_type, W, A_q8_1, Y, out_dtype, mode, bias, M, N, K);
  if (rc != IFX_OK) return rc;
  const hipStream_t s = static_cast<hipStream_t>(stream);
  const bool f16 = out_dtype == IFX_OUT_F16;
  const Route r = route(quant_type, M, K, N, f16, false, !ordered && mode == IFX_ACCUM);
  int wrc = IFX_OK;
  switch (r) {
  case Route::F16Gemm:
    return status_of(ifx::launch_gemm_f16(quant_type, W, A_q8_1, nullptr, Y, bias, f16, M, N, K, mode, 0, s));
  case Route::Gemv:
    return status_of(ifx::launch_gemv(quant_type, W, A_q8_1, Y, bias, f16, M, N, K, mode, s));
  case Route::Lds:
    return status_of(ifx::launch_gemv_lds(1, &W, &Y, &N, bias, A_q8_1, f16, M, K, mode, s));
  case Route::Slot: {
    void *w = split_ws(r, ws, ws_bytes, 1, &N, f16, M, K, ordered, wrc);
    if (wrc != IFX_OK) return wrc;
    return status_of(ifx::launch_gemv_slot(quant_type, 1, &W, &Y, &N, bias, A_q8_1, f16, M, K, mode, s, w));
  }
  case Route::Dq: {
    void *w = split_ws(r, ws, ws_bytes, 1, &N, f16, M, K, ordered, wrc);
    if (wrc != IFX_OK) return wrc;
    // tiled weights: fp16 outputs split only through the workspace
    if (f16 && !w && !ifx::gemv_dq_f16_unsplit(1, &N, M, K)) return IFX_BAD_GEOMETRY;
    return status_of(ifx::launch_gemv_dq(quant_type, 1, &W, &Y, &N, bias, A_q8_1, f16, M, K, mode, 0, s, w));
  }
  case Route::Skinny:
    return status_of(ifx::launch_mmq_skinny(quant_type, 1, &W, &Y, &N, bias, A_q8_1, f16, M, K, mode, s));
  case Route::Mmvq:
    return status_of(ifx::launch_mmvq(quant_type, 1, &W, &Y, &N, bias, A_q8_1, f16, M, K, mode, s));
  default:
    return status_of(ifx::launch_gemm_mfma(quant_type, W, A_q8_1, Y, bias, f16, M, N, K, mode, s));
  }
}

int grouped_impl(int quant_type, int count, const void *const *W, void *const *Y, const int *N,
                 const void *A_q8_1, int out_dtype, int mode, int M, int K, void *stream, void *ws,
                 int64_t ws_bytes, bool ordered) {
  if (!W || !Y || !N) return IFX_NULL_POINTER;
  if (count < 1 || count > 3) return IFX_BAD_GEOMETRY;
  if (mode == IFX_BIAS) return IFX_BAD_GEOMETRY;
  for (int i = 0; i < count; ++i) {
    const int rc = check_gemm_args(quant_type, W[i], A_q8_1, Y[i], out_dtype, mode, nullptr, M,
                                   N[i], K);
    if (rc != IFX_OK) return rc;
  }
  const hipStream_t s = static_cast<hipStream_t>(stream);
  const bool f16 = out_dtype == IFX_OUT_F16;
  int n_total = 0;
  for (int i = 0; i < count; ++i) n_total += N[i];
  const Route r = route(quant_type, M, K, n_total, f16, true, !ordered && mode == IFX_ACCUM);
  int wrc = IFX_OK;
  switch (r) {
  case Route::Gemv:
    return status_of(
        ifx::launch_gemv_grouped(quant_type, count, W, Y, N, A_q8_1, f16, M, K, mode, s));
  case Route::Lds:
    return status_of(ifx::launch_gemv_lds(count, W, Y, N, nullptr, A_q8_1, f16, M, K, mode, s));
  case Route::Slot: {
    void *w = split_ws(r, ws, ws_bytes, count, N, f16, M, K, ordered, wrc);
    if (wrc != IFX_OK) return wrc;
    return status_of(ifx::launch_gemv_slot(quant_type, count, W, Y, N, nullptr, A_q8_1, f16, M, K,
                                           mode, s, w));
  }
  case Route::Dq: {
    void *w = split_ws(r, ws, ws_bytes, count, N, f16, M, K, ordered, wrc);
    if (wrc != IFX_OK) return wrc;
    if (f16 && !w && !ifx::gemv_dq_f16_unsplit(count, N, M, K))  // tiled weights
      return IFX_BAD_GEOMETRY;
    return status_of(ifx::launch_gemv_dq(quant_type, count, W, Y, N, nullptr, A_q8_1, f16, M, K,
                                         mode, 0, s, w));
  }
  case Route::Skinny:
    return status_of(ifx::launch_mmq_skinny(quant_type, count, W, Y, N, nullptr, A_q8_1, f16, M,
                                            K, mode, s));
  case Route::Mmvq:
    return status_of(ifx::launch_mmvq(quant_type, count, W, Y, N, nullptr, A_q8_1, f16, M, K,
                                      mode, s));
  default:
    break;
  }
  // batched decode and prefill: one launch per projection (each fills the chip)
  for (int i = 0; i < count; ++i) {
    const int rc = qgemv_impl(quant_type, W[i], A_q8_1, Y[i], out_dtype, mode, nullptr, M, N[i],
                              K, stream, ws, ws_bytes, ordered);
    if (rc != IFX_OK) return rc;
  }
  return IFX_OK;
}

}  // namespace


extern "C" {


int ifx_block_bytes(int quant_type) {
  switch (quant_type) {
  case IFX_TYPE_Q4_K: return ifx::kQ4KBytes;
  case IFX_TYPE_Q5_K: return ifx::kQ5KBytes;
  case IFX_TYPE_Q6_K: return ifx::kQ6KBytes;
  case IFX_TYPE_Q8_K: return ifx::kQ8KBytes;
  case IFX_TYPE_Q8_0: return ifx::kQ8_0Bytes;
  case IFX_TYPE_Q8_1: return ifx::kQ8_1Bytes;
  case IFX_TYPE_Q8_0_R: return ifx::kQ8_0Bytes;
  case IFX_TYPE_Q6_K_R: case IFX_TYPE_Q6_K_T: return ifx::kQ6KBytes;
  case IFX_TYPE_Q4_K_T: return ifx::kQ4KBytes;
  case IFX_TYPE_Q8_0_T: return 8 * ifx::kQ8_0Bytes;  // the 256 values of a tile row
  default: return 0;
  }
}

int ifx_block_elems(int quant_type) {
  switch (quant_type) {
  case IFX_TYPE_Q4_K: case IFX_TYPE_Q5_K: case IFX_TYPE_Q6_K: case IFX_TYPE_Q8_K:
  case IFX_TYPE_Q6_K_R: case IFX_TYPE_Q4_K_T: case IFX_TYPE_Q6_K_T: case IFX_TYPE_Q8_0_T: return 256;
  case IFX_TYPE_Q8_0: case IFX_TYPE_Q8_1: case IFX_TYPE_Q8_0_R: return 32;
  default: return 0;
  }
}

const char *ifx_status_string(int status) {
  switch (status) {
  case IFX_OK: return "ok";
  case IFX_UNSUPPORTED_TYPE: return "unsupported quant type";
  case IFX_BAD_GEOMETRY: return "bad geometry or argument";
  case IFX_NULL_POINTER: return "null pointer";
  case IFX_DISABLED: return "fused path disabled by policy";
  case IFX_SCRATCH_LIMIT: return "shape exceeds the static scratch of the no-alloc entry";
  default: return status < 0 ? hipGetErrorString(static_cast<hipError_t>(-status)) : "unknown";
  }
}

int ifx_supports(int quant_type, int M, int N, int K) {
  if (!is_weight_type(quant_type)) return 0;
  if (M <= 0 || N <= 0 || K <= 0 || K % ifx_block_elems(quant_type)) return 0;
  if (gemv_only(quant_type) && M > kMaxGemvOnlyM) return 0;
  if (row_split(quant_type) && M > kMaxRowSplitM) return 0;
  if (tiled(quant_type) && M > kMaxTiledM) return 0;
  return buffers_fit(quant_type, M, N, K) ? 1 : 0;
}

int ifx_kernel_family(int quant_type, int M, int N, int K) {
  if (!ifx_supports(quant_type, M, N, K)) return 0;
  switch (route(quant_type, M, K, N, false, false)) {
  case Route::Gemv: case Route::Lds: return 1;
  case Route::Slot: case Route::Skinny: case Route::Mmvq: return 2;
  case Route::F16Gemm: return 4;
  case Route::Dq: return 5;
  default: return 3;
  }
}

void ifx_launch_log_begin(int dry_run) {
  ifx::g_log.open = true;
  ifx::g_log.dry = dry_run != 0;
  ifx::g_log.text.clear();
}

const char *ifx_launch_log_end(void) {
  if (!ifx::g_log.open) return "";
  ifx::g_log.open = false;
  ifx::g_log.dry = false;
  return ifx::g_log.text.c_str();
}

int ifx_q8_1_quantize_f32(const float *x, void *q8_1, int M, int K, void *stream) {
  if (!x || !q8_1) return IFX_NULL_POINTER;
  if (M < 0 || K < 0 || K % 32) return IFX_BAD_GEOMETRY;
  return status_of(ifx::launch_quantize_q8_1(x, false, q8_1, M, K,
                                             static_cast<hipStream_t>(stream)));
}

int ifx_q8_1_quantize_f16(const uint16_t *x, void *q8_1, int M, int K, void *stream) {
  if (!x || !q8_1) return IFX_NULL_POINTER;
  if (M < 0 || K < 0 || K % 32) return IFX_BAD_GEOMETRY;
  return status_of(ifx::launch_quantize_q8_1(x, true, q8_1, M, K,
                                             static_cast<hipStream_t>(stream)));
}

int ifx_rmsnorm_quantize_q8_1(const void *residual, int residual_dtype,
                              const uint16_t *norm_weight, void *q8_1, int M, int K, float eps,
                              void *stream) {
  if (!residual || !norm_weight || !q8_1) return IFX_NULL_POINTER;
  if (residual_dtype != IFX_OUT_F32 && residual_dtype != IFX_OUT_F16) return IFX_BAD_GEOMETRY;
  if (M < 0 || K <= 0 || K % 32 || !(eps >= 0.0f)) return IFX_BAD_GEOMETRY;
  return status_of(ifx::launch_rmsnorm_quantize_q8_1(residual, residual_dtype == IFX_OUT_F16,
                                                     norm_weight, q8_1, M, K, eps,
                                                     static_cast<hipStream_t>(stream)));
}

int ifx_silu_mul_quantize_q8_1(const void *gate, const void *up, int dtype, void *q8_1, int M,
                               int K, void *stream) {
  if (!gate || !up || !q8_1) return IFX_NULL_POINTER;
  if (dtype != IFX_OUT_F32 && dtype != IFX_OUT_F16) return IFX_BAD_GEOMETRY;
  if (M < 0 || K < 0 || K % 32) return IFX_BAD_GEOMETRY;
  return status_of(ifx::launch_silu_mul_quantize_q8_1(gate, up, dtype == IFX_OUT_F16, q8_1, M, K,
                                                      static_cast<hipStream_t>(stream)));
}

int ifx_quantize_rows_symmetric(const void *x, int dtype, int8_t *codes, float *row_scales, int M,
                                int K, void *stream) {
  if (!x || !codes || !row_scales) return IFX_NULL_POINTER;
  if (dtype != IFX_OUT_F32 && dtype != IFX_OUT_F16 && dtype != IFX_IN_BF16) return IFX_BAD_GEOMETRY;
  if (M < 0 || K <= 0) return IFX_BAD_GEOMETRY;
  return status_of(ifx::launch_quantize_rows_sym(x, nullptr, dtype, codes, row_scales, M, K,
                                                 static_cast<hipStream_t>(stream)));
}

int ifx_silu_mul_quantize_rows_symmetric(const void *gate, const void *up, int dtype,
                                         int8_t *codes, float *row_scales, int M, int K,
                                         void *stream) {
  if (!gate || !up || !codes || !row_scales) return IFX_NULL_POINTER;
  if (dtype != IFX_OUT_F32 && dtype != IFX_OUT_F16 && dtype != IFX_IN_BF16) return IFX_BAD_GEOMETRY;
  if (M < 0 || K <= 0) return IFX_BAD_GEOMETRY;
  return status_of(ifx::launch_quantize_rows_sym(gate, up, dtype, codes, row_scales, M, K,
                                                 static_cast<hipStream_t>(stream)));
}

int ifx_qgemv_packed(int quant_type, int count, const void *const *W, void *const *Y,
                     const int *N, const int8_t *codes, const float *row_scales, int M, int K,
                     void *stream) {
  if (quant_type != IFX_TYPE_Q4_K && quant_type != IFX_TYPE_Q6_K && quant_type != IFX_TYPE_Q8_0 &&
      quant_type != IFX_TYPE_Q8_K)
    return IFX_UNSUPPORTED_TYPE;
  if (!W || !Y || !N || !codes || !row_scales) return IFX_NULL_POINTER;
  if (count < 1 || count > 3 || M < 0 || !ifx::gemv_packed_fits(quant_type, K))
    return IFX_BAD_GEOMETRY;
  // 32-bit buffer ranges: each weight tensor and the activation rows
  if (static_cast<int64_t>(M) * K >= (int64_t{1} << 32)) return IFX_BAD_GEOMETRY;
  for (int i = 0; i < count; ++i) {
    if (!W[i] || !Y[i]) return IFX_NULL_POINTER;
    if (N[i] <= 0 || static_cast<int64_t>(N[i]) * ifx::row_bytes(quant_type, K) >= (int64_t{1} << 32))
      return IFX_BAD_GEOMETRY;
  }
  return status_of(ifx::launch_gemv_packed(quant_type, count, W, Y, N, codes, row_scales, M, K,
                                           static_cast<hipStream_t>(stream)));
}

int ifx_qgemv(int quant_type, const void *W, const void *A_q8_1, void *Y, int out_dtype, int mode,
              const void *bias, int M, int N, int K, void *stream) {
  return qgemv_impl(quant_type, W, A_q8_1, Y, out_dtype, mode, bias, M, N, K, stream, nullptr, 0,
                    false);
}

int ifx_qgemv_ws(int quant_type, const void *W, const void *A_q8_1, void *Y, int out_dtype,
                 int mode, const void *bias, int M, int N, int K, void *workspace,
                 int64_t workspace_bytes, void *stream) {
  if (!workspace && workspace_bytes != 0) return IFX_NULL_POINTER;
  return qgemv_impl(quant_type, W, A_q8_1, Y, out_dtype, mode, bias, M, N, K, stream, workspace,
                    workspace_bytes, true);
}

int ifx_qgemv_grouped(int quant_type, int count, const void *const *W, void *const *Y,
                      const int *N, const void *A_q8_1, int out_dtype, int mode, int M, int K,
                      void *stream) {
  return grouped_impl(quant_type, count, W, Y, N, A_q8_1, out_dtype, mode, M, K, stream, nullptr,
                      0, false);
}

int ifx_qgemv_grouped_ws(int quant_type, int count, const void *const *W, void *const *Y,
                         const int *N, const void *A_q8_1, int out_dtype, int mode, int M, int K,
                         void *workspace, int64_t workspace_bytes, void *stream) {
  if (!workspace && workspace_bytes != 0) return IFX_NULL_POINTER;
  return grouped_impl(quant_type, count, W, Y, N, A_q8_1, out_dtype, mode, M, K, stream,
                      workspace, workspace_bytes, true);
}

int64_t ifx_qgemv_workspace_bytes(int quant_type, int count, const int *N, int out_dtype, int M,
                                  int K) {
  if (!N || count < 1 || count > 3 || !is_weight_type(quant_type) || M <= 0 || K <= 0 ||
      K % ifx_block_elems(quant_type))
    return 0;
  int n_total = 0;
  for (int i = 0; i < count; ++i) {
    if (N[i] <= 0) return 0;
    n_total += N[i];
  }
  const bool f16 = out_dtype == IFX_OUT_F16;
  switch (route(quant_type, M, K, n_total, f16, count > 1)) {
  case Route::Slot: return ifx::gemv_slot_workspace_bytes(count, N, f16, M, K);
  case Route::Dq: return ifx::gemv_dq_workspace_bytes(count, N, f16, M, K);
  default: return 0;
  }
}

int ifx_qgemv_grouped_rmsnorm(int quant_type, int count, const void *const *W, void *const *Y,
                              const int *N, const void *residual, int residual_dtype,
                              const uint16_t *norm_weight, float eps, int out_dtype, int mode,
                              int M, int K, void *stream) {
  if (!W || !Y || !N || !residual) return IFX_NULL_POINTER;
  if (count < 1 || count > 3) return IFX_BAD_GEOMETRY;
  if (mode != IFX_STORE && mode != IFX_ACCUM) return IFX_BAD_GEOMETRY;
  if (residual_dtype != IFX_OUT_F32 && residual_dtype != IFX_OUT_F16) return IFX_BAD_GEOMETRY;
  if (!(eps >= 0.0f)) return IFX_BAD_GEOMETRY;
  for (int i = 0; i < count; ++i) {
    // geometry and 32-bit range checks of the GEMV (the activation pointer
    // stands in for the Q8_1 tensor the kernel builds in LDS)
    const int rc = check_gemm_args(quant_type, W[i], residual, Y[i], out_dtype, mode, nullptr, M,
                                   N[i], K);
    if (rc != IFX_OK) return rc;
  }
  if (quant_type != IFX_TYPE_Q4_K || M > 2 ||
      static_cast<int64_t>(M) * ifx::split_row_bytes(K) > 65536)  // the LDS activation rows
    return IFX_BAD_GEOMETRY;
  return status_of(ifx::launch_gemv_rmsnorm(count, W, Y, N, residual,
                                            residual_dtype == IFX_OUT_F16, norm_weight, eps,
                                            out_dtype == IFX_OUT_F16, M, K, mode,
                                            static_cast<hipStream_t>(stream)));
}

namespace {

// The fused gate/up/SiLU launches: M <= 2 the v_dot4 GEMV; 3 <= M <= 8
// (Q4_K / Q6_K) the slot-packed MFMA GEMV; tiled rows up to M = 32 the GEMV
// the grouped gate+up launch runs (route()); the rest up to M = 32 the
// fp16-dequant MFMA GEMV, whose K split needs the pair's ordered-split
// workspace unless the split is 1.  Whole Q8_1 blocks of outputs only.
enum class SwKernel { None, Gemv, Slot, Dq };
SwKernel swiglu_kernel(int qt, int M, int N, int K) {
  const int max_m = tiled(qt) ? 0 : (qt == IFX_TYPE_Q4_K && K <= 2048) ? IFX_SWIGLU_MAX_M : 2;
  if (M < 1) return SwKernel::None;
  if (M <= max_m) return SwKernel::Gemv;
  if (tiled(qt)) {
    if (M > 32) return SwKernel::None;
    if (route(qt, M, K, 2 * N, false, true) == Route::Slot)
      return ifx::gemv_slot_fits(qt, M, K) ? SwKernel::Slot : SwKernel::None;
    return ifx::gemv_dq_fits(qt, M, K) ? SwKernel::Dq : SwKernel::None;
  }
  if (M <= kMaxSlotM && ifx::gemv_slot_fits(qt, M, K)) return SwKernel::Slot;
  return ifx::gemv_dq_fits(qt, M, K) ? SwKernel::Dq : SwKernel::None;
}

int gate_up_silu_impl(int quant_type, const void *W_gate, const void *W_up, const void *A_q8_1,
                      void *H, int h_dtype, void *q8_1_out, int M, int N, int K, void *ws,
                      int64_t ws_bytes, void *stream) {
  if (!W_gate || !W_up || !A_q8_1 || (!H && !q8_1_out)) return IFX_NULL_POINTER;
  if (!is_weight_type(quant_type) || row_split(quant_type)) return IFX_UNSUPPORTED_TYPE;
  if (h_dtype != IFX_OUT_F32 && h_dtype != IFX_OUT_F16) return IFX_BAD_GEOMETRY;
  const SwKernel kern = swiglu_kernel(quant_type, M, N, K);
  const bool slot = kern == SwKernel::Slot, dq = kern == SwKernel::Dq;
  if (kern == SwKernel::None || N % 32 != 0) return IFX_BAD_GEOMETRY;
  // geometry and 32-bit range checks of the GEMV (the output pointer is
  // only checked for presence)
  void *probe_out = H ? H : q8_1_out;
  const int rc = check_gemm_args(quant_type, W_gate, A_q8_1, probe_out, IFX_OUT_F32, IFX_STORE,
                                 nullptr, M, N, K);
  if (rc != IFX_OK) return rc;
  const hipStream_t s = static_cast<hipStream_t>(stream);
  if (slot)
    return status_of(ifx::launch_gemv_slot_swiglu(quant_type, W_gate, W_up, A_q8_1, H,
                                                  h_dtype == IFX_OUT_F16, q8_1_out, M, N, K, s));
  if (dq) {
    if (ifx::gemv_dq_swiglu_splits(M, N, K) > 1) {
      const int NN[2] = {N, N};
      if (!ws) return IFX_BAD_GEOMETRY;  // not handled without the workspace
      if (ws_bytes < ifx::gemv_dq_workspace_bytes(2, NN, false, M, K)) return IFX_BAD_GEOMETRY;
    } else {
      ws = nullptr;
    }
    if (ws_bytes > 0 && reinterpret_cast<uintptr_t>(ws) % 256) return IFX_BAD_GEOMETRY;
    return status_of(ifx::launch_gemv_dq_swiglu(quant_type, W_gate, W_up, A_q8_1, H,
                                                h_dtype == IFX_OUT_F16, q8_1_out, M, N, K, ws, s));
  }
  return status_of(ifx::launch_gemv_swiglu(quant_type, W_gate, W_up, A_q8_1, H,
                                           h_dtype == IFX_OUT_F16, q8_1_out, M, N, K, s));
}

}  // namespace

int ifx_qgemv_gate_up_silu(int quant_type, const void *W_gate, const void *W_up,
                           const void *A_q8_1, void *H, int h_dtype, void *q8_1_out, int M,
                           int N, int K, void *stream) {
  return gate_up_silu_impl(quant_type, W_gate, W_up, A_q8_1, H, h_dtype, q8_1_out, M, N, K,
                           nullptr, 0, stream);
}

int64_t ifx_qgemv_gate_up_silu_workspace_bytes(int quant_type, int M, int N, int K) {
  if (!is_weight_type(quant_type) || row_split(quant_type) || M < 1 || N < 1 || K < 1) return 0;
  if (swiglu_kernel(quant_type, M, N, K) != SwKernel::Dq) return 0;
  if (ifx::gemv_dq_swiglu_splits(M, N, K) <= 1) return 0;
  const int NN[2] = {N, N};
  return ifx::gemv_dq_workspace_bytes(2, NN, false, M, K);
}

int ifx_qgemv_gate_up_silu_ws(int quant_type, const void *W_gate, const void *W_up,
                              const void *A_q8_1, void *H, int h_dtype, void *q8_1_out, int M,
                              int N, int K, void *workspace, int64_t workspace_bytes,
                              void *stream) {
  if (!workspace) return IFX_NULL_POINTER;
  return gate_up_silu_impl(quant_type, W_gate, W_up, A_q8_1, H, h_dtype, q8_1_out, M, N, K,
                           workspace, workspace_bytes, stream);
}

int ifx_qgemv_gate_up_silu_rmsnorm(int quant_type, const void *W_gate, const void *W_up,
                                   const void *residual, int residual_dtype,
                                   const uint16_t *norm_weight, float eps, void *H, int h_dtype,
                                   void *q8_1_out, int M, int N, int K, void *stream) {
  if (!W_gate || !W_up || !residual || !norm_weight || (!H && !q8_1_out)) return IFX_NULL_POINTER;
  if (!is_weight_type(quant_type)) return IFX_UNSUPPORTED_TYPE;
  if (h_dtype != IFX_OUT_F32 && h_dtype != IFX_OUT_F16) return IFX_BAD_GEOMETRY;
  if (residual_dtype != IFX_OUT_F32 && residual_dtype != IFX_OUT_F16) return IFX_BAD_GEOMETRY;
  if (!(eps >= 0.0f)) return IFX_BAD_GEOMETRY;
  void *probe_out = H ? H : q8_1_out;
  const int rc = check_gemm_args(quant_type, W_gate, residual, probe_out, IFX_OUT_F32, IFX_STORE,
                                 nullptr, M, N, K);
  if (rc != IFX_OK) return rc;
  // the wide Q4_K kernel only: one row's slices fit half a wave
  if (quant_type != IFX_TYPE_Q4_K || M > IFX_SWIGLU_MAX_M || N % 32 != 0 || K > 2048)
    return IFX_BAD_GEOMETRY;
  return status_of(ifx::launch_gemv_swiglu_rmsnorm(W_gate, W_up, residual,
                                                   residual_dtype == IFX_OUT_F16, norm_weight, eps,
                                                   H, h_dtype == IFX_OUT_F16, q8_1_out, M, N, K,
                                                   static_cast<hipStream_t>(stream)));
}

int ifx_qgemm_prefill(int quant_type, const void *W, const void *A_q8_1, void *Y, int out_dtype,
                      int mode, const void *bias, int M, int N, int K, void *stream) {
  const int rc = check_gemm_args(quant_type, W, A_q8_1, Y, out_dtype, mode, bias, M, N, K);
  if (rc != IFX_OK) return rc;
  if (gemv_only(quant_type) || repacked(quant_type)) return IFX_UNSUPPORTED_TYPE;  // no MFMA kernel for the type
  const bool f16 = out_dtype == IFX_OUT_F16;
  const hipStream_t s = static_cast<hipStream_t>(stream);
  if (use_f16_gemm(quant_type, M, K))
    return status_of(ifx::launch_gemm_f16(quant_type, W, A_q8_1, nullptr, Y, bias, f16, M, N, K, mode, 0, s));
  return status_of(ifx::launch_gemm_mfma(quant_type, W, A_q8_1, Y, bias, f16, M, N, K, mode, s));
}

// The fp16 copy pays where many weight tiles share it: measured at M = 512,
// Q4_K 27648 x 5120 (108 tiles of 256 columns) 190 -> 162 us, Q6_K
// 5120 x 27648 (20 tiles) 234 -> 250 us.
constexpr int kMinWorkspaceN = 16384;

int64_t ifx_qgemm_prefill_workspace_bytes(int quant_type, int M, int N, int K) {
  if (!is_weight_type(quant_type) || gemv_only(quant_type) || repacked(quant_type) || M <= 0 ||
      N <= 0 || K <= 0)
    return 0;
  if (!use_f16_gemm(quant_type, M, K) || !ifx::gemm_f16_fits(quant_type, K) || N < kMinWorkspaceN)
    return 0;
  return ifx::gemm_f16_workspace_bytes(M, K);
}

int ifx_qgemm_prefill_ws(int quant_type, const void *W, const void *A_q8_1, void *Y, int out_dtype,
                         int mode, const void *bias, int M, int N, int K, void *workspace,
                         int64_t workspace_bytes, void *stream) {
  const int rc = check_gemm_args(quant_type, W, A_q8_1, Y, out_dtype, mode, bias, M, N, K);
  if (rc != IFX_OK) return rc;
  if (gemv_only(quant_type) || repacked(quant_type)) return IFX_UNSUPPORTED_TYPE;
  const int64_t need = ifx_qgemm_prefill_workspace_bytes(quant_type, M, N, K);
  if (need == 0 || !workspace)
    return ifx_qgemm_prefill(quant_type, W, A_q8_1, Y, out_dtype, mode, bias, M, N, K, stream);
  if (workspace_bytes < need || reinterpret_cast<uintptr_t>(workspace) % 16 != 0)
    return IFX_BAD_GEOMETRY;
  return status_of(ifx::launch_gemm_f16(quant_type, W, A_q8_1, workspace, Y, bias,
                                        out_dtype == IFX_OUT_F16, M, N, K, mode, 0,
                                        static_cast<hipStream_t>(stream)));
}

// The ordered prefill's workspace: the fp16 activation copy of
// ifx_qgemm_prefill_ws (when the shape uses one), 256-byte aligned, then
// the K splits' slots (when the launch splits K).
int64_t ordered_a16_bytes(int quant_type, int M, int N, int K) {
  return (ifx_qgemm_prefill_workspace_bytes(quant_type, M, N, K) + 255) / 256 * 256;
}
int64_t ordered_slot_bytes(int quant_type, int out_dtype, int M, int N, int K) {
  if (!is_weight_type(quant_type) || gemv_only(quant_type) || repacked(quant_type) || M <= 0 ||
      N <= 0 || K <= 0 || !use_f16_gemm(quant_type, M, K) || !ifx::gemm_f16_fits(quant_type, K))
    return 0;
  return ifx::gemm_f16_slot_bytes(out_dtype == IFX_OUT_F16, M, N, K);
}

int64_t ifx_qgemm_prefill_ordered_workspace_bytes(int quant_type, int out_dtype, int M, int N,
                                                  int K) {
  const int64_t slots = ordered_slot_bytes(quant_type, out_dtype, M, N, K);
  const int64_t a16 = ifx_qgemm_prefill_workspace_bytes(quant_type, M, N, K);
  return slots ? ordered_a16_bytes(quant_type, M, N, K) + slots : a16;
}

int ifx_qgemm_prefill_ordered(int quant_type, const void *W, const void *A_q8_1, void *Y,
                              int out_dtype, int mode, const void *bias, int M, int N, int K,
                              void *workspace, int64_t workspace_bytes, void *stream) {
  const int rc = check_gemm_args(quant_type, W, A_q8_1, Y, out_dtype, mode, bias, M, N, K);
  if (rc != IFX_OK) return rc;
  if (gemv_only(quant_type) || repacked(quant_type)) return IFX_UNSUPPORTED_TYPE;
  const int64_t slots = ordered_slot_bytes(quant_type, out_dtype, M, N, K);
  if (slots == 0)  // no K split: the workspace entry is already deterministic
    return ifx_qgemm_prefill_ws(quant_type, W, A_q8_1, Y, out_dtype, mode, bias, M, N, K,
                                workspace, workspace_bytes, stream);
  if (!workspace) return IFX_NULL_POINTER;
  const int64_t a16 = ordered_a16_bytes(quant_type, M, N, K);
  if (workspace_bytes < a16 + slots || reinterpret_cast<uintptr_t>(workspace) % 256 != 0)
    return IFX_BAD_GEOMETRY;
  uint8_t *base = static_cast<uint8_t *>(workspace);
  return status_of(ifx::launch_gemm_f16(quant_type, W, A_q8_1, a16 ? base : nullptr, Y, bias,
                                        out_dtype == IFX_OUT_F16, M, N, K, mode, 0,
                                        static_cast<hipStream_t>(stream),
                                        reinterpret_cast<float *>(base + a16)));
}

int ifx_qgemm_prefill_noalloc(int quant_type, const void *W, const void *A_q8_1, void *Y,
                              int out_dtype, int mode, const void *bias, int M, int N, int K,
                              void *stream) {
  const int rc = check_gemm_args(quant_type, W, A_q8_1, Y, out_dtype, mode, bias, M, N, K);
  if (rc != IFX_OK) return rc;
  if (gemv_only(quant_type) || repacked(quant_type)) return IFX_UNSUPPORTED_TYPE;
  const int64_t need = ifx_qgemm_prefill_workspace_bytes(quant_type, M, N, K);
  if (need == 0)
    return ifx_qgemm_prefill(quant_type, W, A_q8_1, Y, out_dtype, mode, bias, M, N, K, stream);
  if (need > IFX_NOALLOC_SCRATCH_BYTES) return IFX_SCRATCH_LIMIT;
  void *ws = reinterpret_cast<void *>(uintptr_t{256});  // dry run: never dereferenced
  if (!ifx::dry_run()) {
    const hipError_t e = ifx::scratch_address(&ws);
    if (e != hipSuccess) return status_of(e);
  }
  return status_of(ifx::launch_gemm_f16(quant_type, W, A_q8_1, ws, Y, bias,
                                        out_dtype == IFX_OUT_F16, M, N, K, mode, 0,
                                        static_cast<hipStream_t>(stream)));
}

int ifx_qgemm_prefill_kernel(int quant_type, const void *W, const void *A_q8_1, void *Y,
                             int out_dtype, int mode, const void *bias, int M, int N, int K,
                             int kernel, int splits, void *stream) {
  const int rc = check_gemm_args(quant_type, W, A_q8_1, Y, out_dtype, mode, bias, M, N, K);
  if (rc != IFX_OK) return rc;
  if (gemv_only(quant_type) || repacked(quant_type)) return IFX_UNSUPPORTED_TYPE;
  const bool f16 = out_dtype == IFX_OUT_F16;
  const hipStream_t s = static_cast<hipStream_t>(stream);
  if (kernel == IFX_PREFILL_INT8)
    return status_of(ifx::launch_gemm_mfma(quant_type, W, A_q8_1, Y, bias, f16, M, N, K, mode, s));
  if (kernel == IFX_DECODE_DQ_F16) {
    if (!ifx::gemv_dq_fits(quant_type, M, K) || splits < 0) return IFX_BAD_GEOMETRY;
    if (f16 && !ifx::gemv_dq_fits_f16(M, K)) return IFX_BAD_GEOMETRY;
    return status_of(ifx::launch_gemv_dq(quant_type, 1, &W, &Y, &N, bias, A_q8_1, f16, M, K, mode,
                                         splits, s));
  }
  if (kernel != IFX_PREFILL_F16 || splits < 0) return IFX_BAD_GEOMETRY;
  if (!ifx::gemm_f16_fits(quant_type, K)) return IFX_BAD_GEOMETRY;
  return status_of(ifx::launch_gemm_f16(quant_type, W, A_q8_1, nullptr, Y, bias, f16, M, N, K, mode, splits, s));
}

int64_t ifx_repacked_bytes(int quant_type, int64_t n_rows, int K) {
  const int rt = quant_type == IFX_TYPE_Q8_0 ? IFX_TYPE_Q8_0_R
                 : quant_type == IFX_TYPE_Q6_K ? IFX_TYPE_Q6_K_R : 0;
  if (!rt || n_rows < 0 || K <= 0 || K % ifx_block_elems(quant_type)) return 0;
  return n_rows * static_cast<int64_t>(ifx::row_bytes(rt, K));
}

int ifx_repack(int quant_type, const void *W, void *W_out, int64_t n_rows, int K, void *stream) {
  if (!W || !W_out) return IFX_NULL_POINTER;
  if (quant_type != IFX_TYPE_Q8_0 && quant_type != IFX_TYPE_Q6_K) return IFX_UNSUPPORTED_TYPE;
  if (n_rows < 0 || K <= 0 || K % ifx_block_elems(quant_type)) return IFX_BAD_GEOMETRY;
  if (ifx_repacked_bytes(quant_type, n_rows, K) >= (int64_t{1} << 32) ||
      n_rows * (K / ifx_block_elems(quant_type)) * static_cast<int64_t>(ifx_block_bytes(quant_type)) >=
          (int64_t{1} << 32))
    return IFX_BAD_GEOMETRY;  // the GEMV addresses rows with 32-bit offsets
  return status_of(ifx::launch_repack(quant_type, W, W_out, n_rows, K, static_cast<hipStream_t>(stream)));
}

int64_t ifx_tiled_bytes(int quant_type, int64_t n_rows, int K) {
  const int tt = quant_type == IFX_TYPE_Q4_K ? IFX_TYPE_Q4_K_T
                 : quant_type == IFX_TYPE_Q6_K ? IFX_TYPE_Q6_K_T
                 : quant_type == IFX_TYPE_Q8_0 ? IFX_TYPE_Q8_0_T : 0;
  if (!tt || n_rows < 0 || K <= 0 || K % 256) return 0;
  return (n_rows + 31) / 32 * 32 * static_cast<int64_t>(ifx::row_bytes(tt, K));
}

int ifx_repack_tiled(int quant_type, const void *W, void *W_out, int64_t n_rows, int K,
                     void *stream) {
  if (!W || !W_out) return IFX_NULL_POINTER;
  if (quant_type != IFX_TYPE_Q4_K && quant_type != IFX_TYPE_Q6_K && quant_type != IFX_TYPE_Q8_0)
    return IFX_UNSUPPORTED_TYPE;
  if (n_rows < 0 || K <= 0 || K % 256) return IFX_BAD_GEOMETRY;
  if (ifx_tiled_bytes(quant_type, n_rows, K) >= (int64_t{1} << 32))
    return IFX_BAD_GEOMETRY;  // the GEMVs address tiles with 32-bit offsets
  return status_of(ifx::launch_repack_tiled(quant_type, W, W_out, n_rows, K,
                                            static_cast<hipStream_t>(stream)));
}

namespace {
int64_t align256(int64_t x) { return (x + 255) / 256 * 256; }
// The row-major section of a down-projection MMQ layout: the row-split copy
// for Q6_K / Q8_0, the raw rows for Q4_K (already 16-byte aligned).
int mmq_row_type(int qt) {
  return qt == IFX_TYPE_Q4_K ? IFX_TYPE_Q4_K
         : qt == IFX_TYPE_Q6_K ? IFX_TYPE_Q6_K_R
         : qt == IFX_TYPE_Q8_0 ? IFX_TYPE_Q8_0_R : 0;
}
int mmq_tiled_type(int qt) {
  return qt == IFX_TYPE_Q4_K ? IFX_TYPE_Q4_K_T
         : qt == IFX_TYPE_Q6_K ? IFX_TYPE_Q6_K_T
         : qt == IFX_TYPE_Q8_0 ? IFX_TYPE_Q8_0_T : 0;
}
int64_t mmq_rows_bytes(int qt, int64_t rows, int cols) {
  return qt == IFX_TYPE_Q4_K ? rows * static_cast<int64_t>(ifx::row_bytes(IFX_TYPE_Q4_K, cols))
                             : ifx_repacked_bytes(qt, rows, cols);
}
// The ordered-split workspace a layout carries: the largest any tiled
// launch of 3..32 batch rows asks for (fp32 and fp16 outputs plan alike).
int64_t mmq_ws_bytes(int qt, int64_t rows, int cols) {
  if (rows > (1 << 30)) return 0;
  const int N = static_cast<int>(rows);
  int64_t most = 0;
  for (int M = kMaxRowSplitM + 1; M <= kMaxTiledM; ++M)
    most = std::max(most, ifx_qgemv_workspace_bytes(mmq_tiled_type(qt), 1, &N, IFX_OUT_F32, M, cols));
  return most;
}
}  // namespace

int64_t ifx_mmq_layout_rows_offset(int quant_type, int64_t rows, int cols) {
  if (!mmq_tiled_type(quant_type) || rows <= 0) return 0;
  return align256(ifx_tiled_bytes(quant_type, rows, cols));
}

int64_t ifx_mmq_layout_ws_offset(int quant_type, int64_t rows, int cols) {
  const int64_t off = ifx_mmq_layout_rows_offset(quant_type, rows, cols);
  if (off == 0) return 0;
  return align256(off + mmq_rows_bytes(quant_type, rows, cols));
}

int64_t ifx_mmq_layout_bytes(int quant_type, int64_t rows, int cols) {
  const int64_t off = ifx_mmq_layout_ws_offset(quant_type, rows, cols);
  if (off == 0) return 0;
  return off + mmq_ws_bytes(quant_type, rows, cols);
}

int ifx_mmq_layout_build(int quant_type, const void *W, void *layout, int64_t rows, int cols,
                         void *stream) {
  if (!W || !layout) return IFX_NULL_POINTER;
  if (!mmq_tiled_type(quant_type)) return IFX_UNSUPPORTED_TYPE;
  if (rows <= 0 || rows > (1 << 30) || cols <= 0 || cols % 256) return IFX_BAD_GEOMETRY;
  if (reinterpret_cast<uintptr_t>(layout) % 256 != 0) return IFX_BAD_GEOMETRY;
  // each section is addressed from its own base with 32-bit offsets
  const int64_t off = ifx_mmq_layout_rows_offset(quant_type, rows, cols);
  const int64_t raw = rows * static_cast<int64_t>(ifx::row_bytes(quant_type, cols));
  if (off >= (int64_t{1} << 32) || mmq_rows_bytes(quant_type, rows, cols) >= (int64_t{1} << 32) ||
      raw >= (int64_t{1} << 32))
    return IFX_BAD_GEOMETRY;
  const hipStream_t s = static_cast<hipStream_t>(stream);
  char *base = static_cast<char *>(layout);
  char *rows_base = base + off;
  hipError_t e = ifx::launch_repack_tiled(quant_type, W, layout, rows, cols, s);
  if (e != hipSuccess) return status_of(e);
  if (quant_type == IFX_TYPE_Q4_K)
    e = ifx::dry_run() ? hipSuccess : hipMemcpyAsync(rows_base, W, raw, hipMemcpyDeviceToDevice, s);
  else
    e = ifx::launch_repack(quant_type, W, rows_base, rows, cols, s);
  if (e != hipSuccess) return status_of(e);
  // the workspace's counters start at zero (a load-time call, never captured)
  const int64_t ws = mmq_ws_bytes(quant_type, rows, cols);
  if (ws > 0 && !ifx::dry_run())
    e = hipMemsetAsync(base + ifx_mmq_layout_ws_offset(quant_type, rows, cols), 0, ws, s);
  return status_of(e);
}

int ifx_qgemv_mmq(int quant_type, const void *layout, const void *A_q8_1, void *Y, int out_dtype,
                  int mode, int M, int N, int K, int ordered, void *stream) {
  if (!layout) return IFX_NULL_POINTER;
  if (!mmq_tiled_type(quant_type)) return IFX_UNSUPPORTED_TYPE;
  if (mode != IFX_STORE && mode != IFX_ACCUM) return IFX_BAD_GEOMETRY;
  if (M <= 0 || M > kMaxTiledM || N <= 0 || K <= 0 || K % 256) return IFX_BAD_GEOMETRY;
  const char *base = static_cast<const char *>(layout);
  if (M <= kMaxRowSplitM)
    return qgemv_impl(mmq_row_type(quant_type), base + ifx_mmq_layout_rows_offset(quant_type, N, K),
                      A_q8_1, Y, out_dtype, mode, nullptr, M, N, K, stream, nullptr, 0, false);
  // fp16 sums are split only through the workspace; fp32 ones on request
  void *ws = nullptr;
  int64_t wsb = 0;
  if (ordered || out_dtype == IFX_OUT_F16) {
    ws = const_cast<char *>(base) + ifx_mmq_layout_ws_offset(quant_type, N, K);
    wsb = mmq_ws_bytes(quant_type, N, K);
    if (wsb == 0) ws = nullptr;
  }
  return qgemv_impl(mmq_tiled_type(quant_type), layout, A_q8_1, Y, out_dtype, mode, nullptr, M, N,
                    K, stream, ws, wsb, ordered || out_dtype == IFX_OUT_F16);
}

int ifx_dequantize(int quant_type, const void *W, void *out, int out_dtype, int64_t n_rows, int K,
                   void *stream) {
  if (!W || !out) return IFX_NULL_POINTER;
  if (!is_weight_type(quant_type) || repacked(quant_type)) return IFX_UNSUPPORTED_TYPE;
  if (out_dtype != IFX_OUT_F32 && out_dtype != IFX_OUT_F16) return IFX_BAD_GEOMETRY;
  if (n_rows < 0 || K <= 0 || K % ifx_block_elems(quant_type)) return IFX_BAD_GEOMETRY;
  if (n_rows * static_cast<int64_t>((K / ifx_block_elems(quant_type)) * ifx_block_bytes(quant_type)) >= (int64_t{1} << 32))
    return IFX_BAD_GEOMETRY;  // buffer offsets are 32-bit
  return status_of(ifx::launch_dequantize(quant_type, W, out, out_dtype == IFX_OUT_F16,
                                          n_rows * static_cast<int64_t>(K),
                                          static_cast<hipStream_t>(stream)));
}

}  // extern "C"
