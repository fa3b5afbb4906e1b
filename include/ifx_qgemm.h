/*
 * ifx_qgemm.h -- C ABI of the MI355X (gfx950) quantized GEMV/GEMM path.
 *
 * Drop-in replacement for the fused GGUF dequant-GEMV/GEMM operators of
 * InferFlux's native backend, class FusedQuantGemm
 * (runtime/backends/cuda/native/fused_quant_gemm.h:47-398).  Plain pointers
 * and sizes only; every device pointer is caller-owned device memory and
 * every call is enqueued on the caller's HIP stream (passed as void*, a
 * hipStream_t; NULL = the default stream).  Nothing here synchronises the
 * host, and the GEMV/GEMM/quantize entry points allocate nothing.
 *
 * Layouts (as in the reference, weight_map.h:17-21 and
 * quantized_weight_map.cpp:379-434):
 *   W  raw GGUF blocks, row-major [N][K/QK]; row n starts at
 *      W + n * (K/QK) * block_bytes.  QK = 256 for Q4_K/Q6_K, 32 for Q8_0.
 *   A  Q8_1 activations [M][K/32], 36-byte blocks {f16 d, f16 s, i8 qs[32]}.
 *   Y  [M][N] row-major, fp32 or fp16.
 *
 * Status codes: 0 = launched; > 0 = not handled, use a fallback (the
 * reference's `false`); < 0 = -(hipError_t) reported by the launch.
 */
#ifndef IFX_QGEMM_H
#define IFX_QGEMM_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* GGUF tensor type ids (runtime/backends/cuda/native/gguf_util.h:48-63). */
enum ifx_quant_type {
  IFX_TYPE_Q8_0 = 8,
  IFX_TYPE_Q8_1 = 9,
  IFX_TYPE_Q4_K = 12,
  IFX_TYPE_Q5_K = 13, /* GEMV kernel family only, M <= 64 (no reference kernel) */
  IFX_TYPE_Q6_K = 14,
  IFX_TYPE_Q8_K = 15, /* GEMV kernel family only, M <= 64 (the reference's limit) */
  /* The row-split layouts ifx_repack writes (this library's own, no GGUF
   * id): each row's block fields in separate 16-byte-aligned sections.
   * ifx_qgemv / ifx_qgemv_grouped at M <= 2 only. */
  IFX_TYPE_Q8_0_R = 108, /* [qs: K bytes][d: K/32 fp16][pad to 16] per row */
  IFX_TYPE_Q6_K_R = 114, /* [ql: K/2][qh: K/4][scales: K/16][d: K/256 fp16][pad to 16] */
  /* The tiled layouts ifx_repack_tiled writes (this library's own): rows in
   * groups of 32, one tile per group and super-block holding the group's
   * super-blocks in the byte order of the MFMA batch kernels' loads.
   * ifx_qgemv / ifx_qgemv_grouped / ifx_qgemv_gate_up_silu at M <= 32. */
  IFX_TYPE_Q8_0_T = 208, /* 8704-byte tiles per 256 values: codes in 16-byte pieces, then d */
  IFX_TYPE_Q4_K_T = 212, /* 4608-byte tiles: 32 headers, then qs in 16-byte pieces */
  IFX_TYPE_Q6_K_T = 214  /* 6720-byte tiles: ql, qh pieces, 32 x scales, 32 x d */
};

enum ifx_status {
  IFX_OK = 0,
  IFX_UNSUPPORTED_TYPE = 1, /* quant type has no kernel              */
  IFX_BAD_GEOMETRY = 2,     /* M, N or K out of range / not a multiple */
  IFX_NULL_POINTER = 3,     /* a required pointer is NULL            */
  IFX_DISABLED = 4,         /* policy disabled the fused path (C++ wrapper) */
  IFX_SCRATCH_LIMIT = 5     /* the shape needs more than the library's static
                               scratch (ifx_qgemm_prefill_noalloc)      */
};

enum ifx_out_dtype { IFX_OUT_F32 = 0, IFX_OUT_F16 = 1 };

enum ifx_out_mode {
  IFX_STORE = 0, /* Y  = W.a                         (GemvQ8_1)            */
  IFX_ACCUM = 1, /* Y += W.a                         (GemvQ8_1Accum[F32])  */
  IFX_BIAS = 2   /* Y  = W.a + bias[n], bias dtype = Y dtype (GemvQ8_1WithBias) */
};

/* Activation quantizer fp32 -> Q8_1, the BASELINE contract.
 * Replaces FusedQuantGemm::QuantizeRowQ8_1 (fused_quant_gemm.h:118-119;
 * kernel fused_dequant_gemv.cuh:597-655).  x [M][K] fp32, K % 32 == 0. */
int ifx_q8_1_quantize_f32(const float *x, void *q8_1, int M, int K, void *stream);

/* Same, fp16 input: the reference's own signature (const half* input). */
int ifx_q8_1_quantize_f16(const uint16_t *x, void *q8_1, int M, int K, void *stream);

/* Fused RMSNorm then Q8_1: per row, rms = 1/sqrt(sum(x^2)/K + eps),
 * y = (x * rms) * norm_weight, quantized as ifx_q8_1_quantize_f32 does.
 * residual [M][K] fp32 or fp16 (residual_dtype: ifx_out_dtype),
 * norm_weight fp16 [K].  Replaces FusedQuantGemm::FusedRmsNormQuantizeQ8_1
 * (both overloads, fused_quant_gemm.h:131-150; kernels
 * fused_dequant_gemv.cuh:736-904).  The square root and division are
 * correctly rounded (the reference uses rsqrtf). */
int ifx_rmsnorm_quantize_q8_1(const void *residual, int residual_dtype,
                              const uint16_t *norm_weight, void *q8_1, int M, int K, float eps,
                              void *stream);

/* Fused SiLU(gate) * up then Q8_1: y = gate / (1 + exp(-gate)) * up.
 * gate, up [M][K], fp32 or fp16 (dtype: ifx_out_dtype).  Replaces
 * FusedQuantGemm::SiluMulQuantizeQ8_1 (fused_quant_gemm.h:121-129; kernel
 * fused_dequant_gemv.cuh:657-734), which reads fp16. */
int ifx_silu_mul_quantize_q8_1(const void *gate, const void *up, int dtype, void *q8_1, int M,
                               int K, void *stream);

/* ifx_qgemv_gate_up_silu with a caller workspace for the fp16-dequant
 * GEMV's K split (M up to 32): workspace_bytes >=
 * ifx_qgemv_gate_up_silu_workspace_bytes(quant_type, M, N, K), 256-byte
 * aligned, zeroed once before first use; every call leaves it zeroed again.
 * Calls that share a workspace must not overlap.  Shapes that do not split
 * ignore it.  No single-call counterpart in the reference (its fused
 * gate/up/SiLU stops at M = 8). */
int ifx_qgemv_gate_up_silu_ws(int quant_type, const void *W_gate, const void *W_up,
                              const void *A_q8_1, void *H, int h_dtype, void *q8_1_out, int M,
                              int N, int K, void *workspace, int64_t workspace_bytes,
                              void *stream);
/* Workspace bytes ifx_qgemv_gate_up_silu_ws needs (0: none). */
int64_t ifx_qgemv_gate_up_silu_workspace_bytes(int quant_type, int M, int N, int K);

/* Per-row symmetric int8 activations, the input format of ifx_qgemv_packed:
 * per row, scale = max|x| / 127 (0 for a zero row), codes =
 * clamp(rint(x / scale), -127, 127) evaluated as x * (1 / scale) in fp32.
 * x [M][K] fp32, fp16 or bf16 (dtype IFX_OUT_F32, IFX_OUT_F16, IFX_IN_BF16);
 * codes [M][K] int8, row_scales [M] fp32.  Replaces
 * cuda_kernel::QuantizeRowsSymmetric (cuda_kernels.cu:309-369). */
#define IFX_IN_BF16 2
int ifx_quantize_rows_symmetric(const void *x, int dtype, int8_t *codes, float *row_scales, int M,
                                int K, void *stream);

/* Same of y = gate / (1 + exp(-gate)) * up.  Replaces
 * cuda_kernel::SiluMulQuantizeRowsSymmetric (cuda_kernels.cu:371-437). */
int ifx_silu_mul_quantize_rows_symmetric(const void *gate, const void *up, int dtype,
                                         int8_t *codes, float *row_scales, int M, int K,
                                         void *stream);

/* GEMV on packed (per-row symmetric int8) activations, fp16 outputs:
 * Y[i][m][n] = fp16(row_scales[m] * sum_k W[i][n][k] * codes[m][k]) for
 * count = 1..3 projections of one quant type (Q4_K, Q6_K, Q8_K: K % 256 == 0;
 * Q8_0: K % 32 == 0), any M >= 0.  Replaces FusedQuantGemm::GemvPacked,
 * GemvPackedPair and GemvPackedTriple (fused_quant_gemm.h:79-107, .cu
 * 1131-1231; kernels fused_dequant_gemv.cuh:80-580).  The reference applies
 * the row scale inside every block; here once per output (results differ by
 * fp32 rounding). */
int ifx_qgemv_packed(int quant_type, int count, const void *const *W, void *const *Y,
                     const int *N, const int8_t *codes, const float *row_scales, int M, int K,
                     void *stream);

/* Quantized GEMV/GEMM y[m][n] (op)= sum_k W[n][k] * a[m][k] for any M >= 1.
 * Replaces FusedQuantGemm::GemvQ8_1 / GemvQ8_1Accum / GemvQ8_1AccumF32 /
 * GemvQ8_1WithBias (fused_quant_gemm.h:171-173, 190-193, 202-205; .cu
 * 2085-2260) and the dispatch DispatchQ8_1Gemv{Q4K,Q6K,Q8_0}
 * (fused_quant_gemm.cu:1705-1738).  The kernel is chosen by M, shape and
 * type (ifx_launch_log_begin names it): M <= 2 the weight-streaming v_dot4
 * GEMV; 3 <= M <= 16 the integer-dot batch kernels (activations in LDS,
 * slot-packed int8 MFMA, LDS-staged int8 MFMA); 17 <= M <= 32 the fp16-
 * dequant MFMA GEMV; larger M the int8 MFMA GEMM, and from M = 33 (Q6_K),
 * 96 (Q4_K) or 128 (Q8_0) on the fp16 MFMA GEMM with in-kernel dequant (the
 * reference's prefill arithmetic).  The reference returns false for M > 64
 * and falls back to FP16 cuBLAS; here every M is handled.
 * out_dtype: ifx_out_dtype.  mode: ifx_out_mode.  bias may be NULL unless
 * mode == IFX_BIAS. */
int ifx_qgemv(int quant_type, const void *W, const void *A_q8_1, void *Y, int out_dtype,
              int mode, const void *bias, int M, int N, int K, void *stream);

/* count (1..3) sibling projections of one quant type that read the same
 * Q8_1 activations, e.g. gate + up or Q + K + V: y_i (op)= W_i . a with
 * W_i [N[i]][K] and Y_i [M][N[i]].  For M <= 2 this is one launch whose
 * workgroups walk the rows of all projections; larger M runs one MFMA
 * launch per projection.  mode: IFX_STORE or IFX_ACCUM (no bias).  W, Y and
 * N are host arrays of count entries.
 * Replaces FusedQuantGemm::GemvQ8_1Pair / GemvQ8_1Triple
 * (fused_quant_gemm.h:272-276, 309-313; kernels mmvq.cuh:1197-1448). */
int ifx_qgemv_grouped(int quant_type, int count, const void *const *W, void *const *Y,
                      const int *N, const void *A_q8_1, int out_dtype, int mode, int M, int K,
                      void *stream);

/* Deterministic variants of ifx_qgemv / ifx_qgemv_grouped with a caller
 * workspace.  Where the chosen kernel splits K over workgroups (the
 * slot-packed MFMA GEMV on narrow long-K launches such as a down projection,
 * the fp16-dequant MFMA GEMV at 17 <= M <= 32 and on tiled weights), each
 * split stores its fp32 partial sums in the workspace and the last
 * workgroup of a tile to finish adds them in split order and writes Y: the
 * bits are the same run to run, and there is no zero-fill launch and no
 * atomic on Y.  Other launches are those of the plain entries, except fp32
 * accumulate launches at 9 <= M <= 16, which the plain entries run on the
 * fp16-dequant GEMV's atomic split and these on the integer kernels without
 * a split.  workspace: at least ifx_qgemv_workspace_bytes bytes, 256-byte
 * aligned; its leading counters must be zero before the first call (zero
 * the buffer once after allocating it) and every call leaves them zero.
 * workspace may be NULL with workspace_bytes 0: launches that need none run
 * as above, the others return IFX_BAD_GEOMETRY.  Calls that share a
 * workspace must not overlap.  No reference counterpart (the reference's
 * split kernels add with fp32 atomics, mmvq.cuh:280-401). */
int ifx_qgemv_ws(int quant_type, const void *W, const void *A_q8_1, void *Y, int out_dtype,
                 int mode, const void *bias, int M, int N, int K, void *workspace,
                 int64_t workspace_bytes, void *stream);
int ifx_qgemv_grouped_ws(int quant_type, int count, const void *const *W, void *const *Y,
                         const int *N, const void *A_q8_1, int out_dtype, int mode, int M, int K,
                         void *workspace, int64_t workspace_bytes, void *stream);
/* Workspace bytes the _ws entries need for count projections of N[i] rows
 * (count = 1 for ifx_qgemv_ws); 0 when the launch does not split K. */
int64_t ifx_qgemv_workspace_bytes(int quant_type, int count, const int *N, int out_dtype, int M,
                                  int K);

/* RMSNorm + Q8_1 fused into the grouped GEMV that consumes it: for each
 * batch row m, a[m] = Q8_1((x[m] * rms(x[m])) * norm_weight), exactly as
 * ifx_rmsnorm_quantize_q8_1 computes it, then y_i (op)= W_i . a as
 * ifx_qgemv_grouped.  norm_weight == NULL: a[m] = Q8_1(x[m]), exactly as
 * ifx_q8_1_quantize_f32/_f16 compute it (the reference's QuantizeRowQ8_1
 * + GemvQ8_1AccumF32 of the O projection, transformer_forward.cu:609-726).  Every workgroup rebuilds a in LDS after issuing its
 * first weight loads, so the producer's launch and the Q8_1 round trip
 * through memory disappear from the decode layer.  residual [M][K] fp32 or
 * fp16 (residual_dtype: ifx_out_dtype), norm_weight fp16 [K] or NULL.  Handles
 * Q4_K, 1 <= M <= 2, M * (80 K/64 + K/8) <= 65536; other shapes return
 * IFX_BAD_GEOMETRY (not handled: use the two calls).  mode: IFX_STORE or
 * IFX_ACCUM.  No reference counterpart as one call: it fuses
 * FusedQuantGemm::FusedRmsNormQuantizeQ8_1 (fused_quant_gemm.h:131-150)
 * with GemvQ8_1Pair / GemvQ8_1Triple (fused_quant_gemm.h:272-276, 309-313),
 * the sequence of transformer_forward.cu:524-559. */
int ifx_qgemv_grouped_rmsnorm(int quant_type, int count, const void *const *W, void *const *Y,
                              const int *N, const void *residual, int residual_dtype,
                              const uint16_t *norm_weight, float eps, int out_dtype, int mode,
                              int M, int K, void *stream);

/* Fused gate/up GEMV with SiLU: h[m][o] = silu(W_gate[o] . a[m]) *
 * (W_up[o] . a[m]), written to H [M][N] (fp32 or fp16, h_dtype; may be
 * NULL) and/or quantized to Q8_1 blocks of 32 consecutive outputs in
 * q8_1_out [M][N/32] (may be NULL; not both), ready for the down
 * projection without a separate quantize launch.  Handles 1 <= M <= 2 and
 * N % 32 == 0 (every type), 3 <= M <= 8 for Q4_K / Q6_K with K % 256 == 0,
 * and M <= 16 on tiled copies (the slot-packed MFMA GEMV: h and its blocks
 * equal ifx_qgemv_grouped + ifx_silu_mul_quantize_q8_1 bit for bit where
 * the grouped launch runs the same geometry); up to M = 32 (Q4_K / Q6_K /
 * Q8_0, raw or tiled, K % 256 == 0) the fp16-dequant MFMA GEMV, whose K split
 * needs a workspace unless it is 1 (then use ifx_qgemv_gate_up_silu_ws; h and
 * its blocks equal ifx_qgemv_grouped_ws + ifx_silu_mul_quantize_q8_1 bit for
 * bit where the grouped launch is the same GEMV); other shapes return
 * IFX_BAD_GEOMETRY (not handled: use those two calls).
 * Replaces FusedQuantGemm::FusedGateUpSiluGemvQ8_1 and
 * FusedGateUpSiluGemvQ8_1WithEpilogue (fused_quant_gemm.h:281-307; kernels
 * mmvq.cuh:1686-2030), whose Q8_1 epilogue writes a per-element scale; this
 * one writes whole Q8_1 blocks. */
int ifx_qgemv_gate_up_silu(int quant_type, const void *W_gate, const void *W_up,
                           const void *A_q8_1, void *H, int h_dtype, void *q8_1_out, int M,
                           int N, int K, void *stream);

/* ifx_qgemv_gate_up_silu with the RMSNorm + Q8_1 producer of its input
 * fused in: a = Q8_1(rmsnorm(residual[m]) * norm_weight) (the arithmetic
 * of ifx_rmsnorm_quantize_q8_1), then h and/or its Q8_1 blocks as above.
 * Handles Q4_K, 1 <= M <= 2, N % 32 == 0 and K <= 2048; other shapes return
 * IFX_BAD_GEOMETRY (not handled: use ifx_rmsnorm_quantize_q8_1 +
 * ifx_qgemv_gate_up_silu).  Replaces the reference's
 * FusedRmsNormQuantizeQ8_1 followed by FusedGateUpSiluGemvQ8_1WithEpilogue
 * (fused_quant_gemm.h:131-150, 281-307), the FFN entry of
 * transformer_forward.cu:2839-2870. */
int ifx_qgemv_gate_up_silu_rmsnorm(int quant_type, const void *W_gate, const void *W_up,
                                   const void *residual, int residual_dtype,
                                   const uint16_t *norm_weight, float eps, void *H, int h_dtype,
                                   void *q8_1_out, int M, int N, int K, void *stream);

/* The prefill GEMM alone, for any M >= 1, fp32 accumulate: the fp16 MFMA
 * GEMM with in-kernel dequant from 33 (Q6_K), 96 (Q4_K) or 128 (Q8_0) rows
 * on, the int8 MFMA GEMM below (see ifx_qgemm_prefill_kernel).  Replaces
 * the reference's dequantize-to-FP16 + cublasGemmEx fallback
 * (quantized_weight_map.cpp:176-233, cublas_gemm.h:47, called at
 * transformer_forward.cu:1479). */
int ifx_qgemm_prefill(int quant_type, const void *W, const void *A_q8_1, void *Y,
                      int out_dtype, int mode, const void *bias, int M, int N, int K,
                      void *stream);

/* Bytes of caller-owned workspace ifx_qgemm_prefill_ws uses at this shape
 * (the fp16 copy of the activations, M x K halves), or 0 when the prefill
 * GEMM at this shape does not use one: below the fp16 GEMM's range, or
 * N < 16384, where too few weight tiles share the copy for it to pay. */
int64_t ifx_qgemm_prefill_workspace_bytes(int quant_type, int M, int N, int K);

/* ifx_qgemm_prefill with a caller-owned workspace (16-byte aligned, at least
 * ifx_qgemm_prefill_workspace_bytes(quant_type, M, N, K) bytes; NULL or a zero
 * requirement: exactly ifx_qgemm_prefill).  The fp16 GEMM then converts the
 * Q8_1 activations to fp16 once, into the workspace, instead of once per
 * weight tile; the results are bit-identical to ifx_qgemm_prefill.  The
 * workspace is in use until the launches on `stream` complete.  A workspace
 * smaller than required or misaligned returns IFX_BAD_GEOMETRY.  It plays
 * the role of the reference's FP16 scratch for the dequantized weights
 * (quantized_weight_map.cpp:176-233), for the activation operand. */
int ifx_qgemm_prefill_ws(int quant_type, const void *W, const void *A_q8_1, void *Y,
                         int out_dtype, int mode, const void *bias, int M, int N, int K,
                         void *workspace, int64_t workspace_bytes, void *stream);

/* Deterministic prefill: ifx_qgemm_prefill_ws whose K split (fp32 outputs
 * of shapes with too few output tiles to fill the GPU, e.g. Q6_K
 * 5120 x 27648 at M = 512: six splits) stores each split's fp32 tile in its
 * own workspace slot and adds the slots in split order in a second launch,
 * with no zero fill and no fp32 atomics: the same bits on every call.
 * Workspace: at least ifx_qgemm_prefill_ordered_workspace_bytes bytes,
 * 256-byte aligned (the fp16 activation copy where the shape uses one, then
 * splits x M x N fp32 slots); it needs no clearing, and calls sharing one
 * must not overlap.  Shapes that do not split run exactly
 * ifx_qgemm_prefill_ws.  No reference counterpart (the reference's prefill
 * GEMM, cublasGemmEx at transformer_forward.cu:1479, does not split K
 * across launches of its own). */
int64_t ifx_qgemm_prefill_ordered_workspace_bytes(int quant_type, int out_dtype, int M, int N,
                                                  int K);
int ifx_qgemm_prefill_ordered(int quant_type, const void *W, const void *A_q8_1, void *Y,
                              int out_dtype, int mode, const void *bias, int M, int N, int K,
                              void *workspace, int64_t workspace_bytes, void *stream);

/* Size of the library's static device scratch (per GPU, held until the
 * process ends) that ifx_qgemm_prefill_noalloc uses as its workspace. */
#define IFX_NOALLOC_SCRATCH_BYTES (16 << 20)

/* ifx_qgemm_prefill_ws with the library's static scratch as the workspace:
 * allocates nothing (no hipMalloc, no allocating library call), so callers
 * that cannot allocate (code under HIP graph capture, tight serving loops,
 * harnesses that forbid it) get the workspace path.  No counterpart in the
 * reference.  Bit-identical to ifx_qgemm_prefill_ws with a caller workspace.
 * A shape whose workspace (ifx_qgemm_prefill_workspace_bytes) exceeds
 * IFX_NOALLOC_SCRATCH_BYTES returns IFX_SCRATCH_LIMIT and launches nothing;
 * a shape that needs no workspace runs exactly ifx_qgemm_prefill.  Every
 * call on one GPU shares that GPU's scratch: calls that overlap on one GPU
 * (concurrent streams, or threads) race and must be serialized by the
 * caller.  The scratch needs no clearing (each call writes all of the part
 * it reads first).  The first call on a device resolves the scratch's
 * address there (hipGetSymbolAddress). */
int ifx_qgemm_prefill_noalloc(int quant_type, const void *W, const void *A_q8_1, void *Y,
                              int out_dtype, int mode, const void *bias, int M, int N, int K,
                              void *stream);

/* The prefill GEMM with an explicit kernel: IFX_PREFILL_INT8 is the
 * integer-exact int8 MFMA GEMM (the MMQ per-block arithmetic of
 * kernels/mmq.cuh:41-835); IFX_PREFILL_F16 dequantizes W (and the Q8_1
 * activations) to fp16 inside the kernel and runs fp16 MFMA with fp32
 * accumulation, the arithmetic of the reference's dequantize + FP16 GEMM
 * prefill path (quantized_weight_map.cpp:176-233, cublas_gemm.h:47); it
 * needs K % 256 == 0 (Q8_0: K % 64 == 0).  IFX_DECODE_DQ_F16 is the
 * decode-batch kernel with the same fp16 arithmetic (1 <= M <= 32,
 * K % 256 == 0).  splits: K split over workgroups
 * for fp32 outputs (0 = chosen from the shape; ignored by the int8 kernel
 * and for fp16 outputs).  ifx_qgemm_prefill picks the kernel by M.  No
 * reference counterpart as a separate entry point (tuning and tests). */
enum ifx_prefill_kernel { IFX_PREFILL_INT8 = 1, IFX_PREFILL_F16 = 2, IFX_DECODE_DQ_F16 = 3 };
int ifx_qgemm_prefill_kernel(int quant_type, const void *W, const void *A_q8_1, void *Y,
                             int out_dtype, int mode, const void *bias, int M, int N, int K,
                             int kernel, int splits, void *stream);

/* Bytes of the row-split copy of n_rows x K Q8_0 or Q6_K weights (0 for
 * another type or a bad K). */
int64_t ifx_repacked_bytes(int quant_type, int64_t n_rows, int K);

/* Load-time repack of raw GGUF Q8_0 / Q6_K rows into the row-split layout
 * IFX_TYPE_Q8_0_R / IFX_TYPE_Q6_K_R (W_out: ifx_repacked_bytes, caller
 * owned, 16-byte aligned).  Their 34- and 210-byte blocks leave rows and
 * fields unaligned; split, every field is read with aligned 16-byte loads
 * that use all their bytes (measured on the 151936 x 2048 Q8_0 LM head: 5.8
 * against 4.7 TB/s for a pure read of either layout).  The row sums are the
 * raw layout's, bit for bit, wherever the GEMV geometry is the same.  The
 * copy serves the M <= 2 GEMV; larger batches need the raw weights.  Plays
 * the role of the reference's load-time re-tiled down-projection copy
 * (BuildDownProjMmqLayout / transform_downproj_mmq_layout,
 * fused_quant_gemm.h:213-234, fused_quant_gemm.cu:573-596, 1966-2032). */
int ifx_repack(int quant_type, const void *W, void *W_out, int64_t n_rows, int K, void *stream);

/* Bytes of the tiled copy of n_rows x K Q4_K, Q6_K or Q8_0 weights: whole
 * groups of 32 rows (0 for another type or K % 256 != 0). */
int64_t ifx_tiled_bytes(int quant_type, int64_t n_rows, int K);

/* Load-time repack of raw GGUF Q4_K / Q6_K / Q8_0 rows (Q8_0: K % 256 == 0)
 * into the tiled layout IFX_TYPE_Q4_K_T / IFX_TYPE_Q6_K_T / IFX_TYPE_Q8_0_T
 * (W_out: ifx_tiled_bytes, caller owned,
 * 16-byte aligned; the rows of a last partial group are written as zeros).
 * The batch kernels (slot-packed int8 MFMA at M <= 8, fp16-dequant MFMA at
 * 9 <= M <= 32) give each lane one weight row, so on raw rows every load
 * instruction touches 32 rows; on tiles it reads one contiguous kilobyte
 * (3B gate 11008 x 2048 at M = 8: 5.7 against 6.8 us; Q6_K down 2048 x
 * 11008: 8.2 against 12.5 us).  Sums are the raw layout's, bit for bit, for
 * the same kernel and split.  The copy serves M <= 32 only (not the M <= 2
 * v_dot4 GEMV, not the prefill GEMM).  Like the row-split copy, it plays
 * the role of the reference's load-time MMQ re-tiling (BuildDownProjMmqLayout,
 * fused_quant_gemm.h:213-234, fused_quant_gemm.cu:573-596, 1966-2032). */
int ifx_repack_tiled(int quant_type, const void *W, void *W_out, int64_t n_rows, int K,
                     void *stream);

/* The down-projection MMQ layout: one caller-owned allocation holding
 *   - at offset 0, the tiled copy of rows x cols Q4_K / Q6_K / Q8_0 weights
 *     (ifx_repack_tiled);
 *   - at ifx_mmq_layout_rows_offset (256-byte aligned), a row-major copy for
 *     the M <= 2 GEMV: the row-split copy (ifx_repack) of Q6_K / Q8_0, the
 *     raw rows of Q4_K;
 *   - at ifx_mmq_layout_ws_offset, the ordered-split workspace of the tiled
 *     launches (zeroed by ifx_mmq_layout_build; every launch leaves it zero).
 * ifx_qgemv_mmq then runs every M in 1..32 on the faster of the two copies
 * (measured on MI355X, 3B down 2048 x 11008 Q6_K: M = 1 6.5 against 7.0 us
 * raw; M = 8 8.2 against 12.4 us raw).  ifx_mmq_layout_bytes: 0 for another
 * type or cols % 256 != 0.  Replaces the copy FusedQuantGemm::
 * BuildDownProjMmqLayout writes (fused_quant_gemm.h:222-224,
 * fused_quant_gemm.cu:573-596, 1966-2026), whose 8-row tile is a layout of
 * the reference's own CUDA kernel. */
int64_t ifx_mmq_layout_bytes(int quant_type, int64_t rows, int cols);
int64_t ifx_mmq_layout_rows_offset(int quant_type, int64_t rows, int cols);
int64_t ifx_mmq_layout_ws_offset(int quant_type, int64_t rows, int cols);
/* Writes the layout from raw GGUF rows W into `layout` (ifx_mmq_layout_bytes,
 * 256-byte aligned), stream ordered.  Allocates nothing. */
int ifx_mmq_layout_build(int quant_type, const void *W, void *layout, int64_t rows, int cols,
                         void *stream);
/* Y (op)= W . a on a layout of N x K weights (quant_type: the GGUF id of the
 * raw weights), 1 <= M <= 32: M <= 2 the v_dot4 GEMV on the row-major copy,
 * 3 <= M <= 32 the batch kernels on the tiles; mode IFX_STORE or IFX_ACCUM.
 * Where the tiled launch splits K over workgroups, ordered != 0 adds the
 * splits in split order through the layout's workspace (bits identical run
 * to run, as ifx_qgemv_ws) and ordered == 0 with fp32 atomics (as
 * ifx_qgemv); fp16 outputs always take the ordered reduction.  Launches
 * that use the layout's workspace must not overlap (one stream, or the
 * caller's ordering).  Replaces FusedQuantGemm::DownProjMmq
 * (fused_quant_gemm.h:213-216, fused_quant_gemm.cu:2034-2080). */
int ifx_qgemv_mmq(int quant_type, const void *layout, const void *A_q8_1, void *Y, int out_dtype,
                  int mode, int M, int N, int K, int ordered, void *stream);

/* Whole-tensor dequantization of n_rows x K weights to fp32 or fp16.
 * Replaces dequantize_q4_k / dequantize_q6_k / dequantize_q8_0
 * (kernels/dequantization.cuh:70-150). */
int ifx_dequantize(int quant_type, const void *W, void *out, int out_dtype, int64_t n_rows,
                   int K, void *stream);

/* 1 if ifx_qgemv handles (quant_type, M, N, K), else 0.  The weights and
 * the Q8_1 activations must each stay below 0xF0000000 bytes and K at most
 * 2^24 (the kernels' 32-bit buffer offsets; every GEMV / GEMM entry returns
 * IFX_BAD_GEOMETRY beyond them).
 * Replaces FusedQuantGemm::SupportsQ8_1Activations (fused_quant_gemm.h:333)
 * combined with ShouldUseFusedPath (fused_quant_gemm.h:388-391). */
int ifx_supports(int quant_type, int M, int N, int K);

/* Kernel family ifx_qgemv runs (quant_type, M, N, K) on: 0 = not supported,
 * 1 = v_dot4 GEMV, 2 = skinny int8 MFMA (decode batches), 3 = tiled int8
 * MFMA, 4 = fp16 MFMA with in-kernel dequant (prefill; M >= 33 Q6_K, 96 Q4_K, 128 Q8_0), 5 = fp16
 * dequant MFMA GEMV (decode batches 17 <= M <= 32).  No
 * reference counterpart (the reference logs the choice,
 * fused_quant_gemm.cu:2104-2117). */
int ifx_kernel_family(int quant_type, int M, int N, int K);

/* Launch log of the calling thread.  ifx_launch_log_begin opens it: every
 * kernel that the entry points called afterwards on this thread launch is
 * recorded by instance name ("k_gemv<12,1,2,1,4,0,2>": kernel name and
 * template arguments as integers, ';'-separated, in launch order).  With
 * dry_run != 0 nothing is launched (no HIP call is made, no pointer is
 * dereferenced; entry points return IFX_OK after validation), so the
 * dispatch of any shape can be inspected on a host without a GPU.
 * ifx_launch_log_end closes the log and returns its text, valid until the
 * next begin on this thread ("" when no log is open).  Replaces the reference's one-time dispatch log
 * (fused_quant_gemm.cu:2104-2117), which names the chosen kernel path. */
void ifx_launch_log_begin(int dry_run);
const char *ifx_launch_log_end(void);

/* Bytes per block / values per block of a quant type (0 if unknown). */
int ifx_block_bytes(int quant_type);
int ifx_block_elems(int quant_type);

/* Human-readable name of a status code. */
const char *ifx_status_string(int status);

#ifdef __cplusplus
}
#endif

#endif /* IFX_QGEMM_H */
