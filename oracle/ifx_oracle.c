/*
 * ifx_oracle.c -- CPU restatement of InferFlux's quantized GEMV/GEMM path.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the checker that the HIP product
 * path is compared against.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load it.  Nothing in inferflux_amd/
 * links, loads or calls it.
 *
 * Every function cites the reference source it restates (paths are relative
 * to the reference repository root; "native/" abbreviates
 * runtime/backends/cuda/native/).
 *
 * Floating-point contract: build with -ffp-contract=off (see Makefile) so
 * every expression rounds exactly as written, in IEEE fp32 unless stated.
 *
 * Pinning status (how each function is checked, tests/test_oracle.py):
 *   f16 encode/decode      exhaustive vs numpy float16 (65536 codes, 2^20+
 *                          float32 inputs incl. ties, subnormals, overflow)
 *   get_scale_min_k4       round trip of all 64x64 (sc, m) pairs through an
 *                          independent 12-byte packer written in the test
 *   dequant q4_k/q6_k/q8_0 hand-built blocks with closed-form answers
 *                          (d=1, sc=1 -> w=q; q6 scale=1 -> w=q-32; ...)
 *   quantize_q8_1          KATs: zero block, one-hot, the reference's
 *                          (i-16)/8 pattern, ties; plus property checks
 *   gemv_exact (fp64)      brute-force numpy dot over the dequantized
 *                          matrix; linearity; zero inputs
 *   gemv_q8_1 (fp32)       against gemv_exact within 1e-3*||y_row||
 *   quantize_rows_symmetric KATs (ties to even, clamp, zero row, amax code
 *                          127), the round-trip bound |x - q*scale| <=
 *                          scale/2, sign symmetry
 *   gemv_packed_exact      equal to gemv_exact on the same values written
 *                          as Q8_1 blocks (power-of-two row scales make both
 *                          formats exact); closed form for constant rows
 *   ggml_cpu_gemv          against gemv_exact within 1e-2*||y_row|| (its
 *                          activation format is Q8_K/Q8_0, not Q8_1).  The
 *                          ggml source is absent from the reference snapshot
 *                          (external/llama.cpp is an empty submodule), so the
 *                          exact ggml bits are "parity unpinned"; only the
 *                          math is pinned.
 */
#include <math.h>
#include <pthread.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define ORC_QK_K 256
#define ORC_QK8 32

/* GGUF tensor type ids: native/gguf_util.h:48-63 */
enum { ORC_Q8_0 = 8, ORC_Q8_1 = 9, ORC_Q4_K = 12, ORC_Q5_K = 13, ORC_Q6_K = 14, ORC_Q8_K = 15 };

/* Block byte sizes: native/kernels/dequantization.cuh:17-49,117-138,156-166 */
enum {
  ORC_Q4_K_BYTES = 144, /* u16 d, u16 dmin, u8 scales[12], u8 qs[128]      */
  ORC_Q5_K_BYTES = 176, /* u16 d, u16 dmin, u8 scales[12], u8 qh[32], u8 qs[128] */
  ORC_Q6_K_BYTES = 210, /* u8 ql[128], u8 qh[64], i8 scales[16], u16 d LAST */
  ORC_Q8_0_BYTES = 34,  /* u16 d, i8 qs[32]                                 */
  ORC_Q8_1_BYTES = 36,  /* u16 d, u16 s (= d*sum(qs)), i8 qs[32]            */
  ORC_Q8_K_BYTES = 292  /* f32 d, i8 qs[256], i16 bsums[16]                 */
};

int orc_block_bytes(int qtype) {
  switch (qtype) {
  case ORC_Q4_K: return ORC_Q4_K_BYTES;
  case ORC_Q5_K: return ORC_Q5_K_BYTES;
  case ORC_Q6_K: return ORC_Q6_K_BYTES;
  case ORC_Q8_0: return ORC_Q8_0_BYTES;
  case ORC_Q8_1: return ORC_Q8_1_BYTES;
  case ORC_Q8_K: return ORC_Q8_K_BYTES;
  default: return 0;
  }
}

int orc_block_elems(int qtype) {
  switch (qtype) {
  case ORC_Q4_K: case ORC_Q5_K: case ORC_Q6_K: case ORC_Q8_K: return ORC_QK_K;
  case ORC_Q8_0: case ORC_Q8_1: return ORC_QK8;
  default: return 0;
  }
}

/* ------------------------------------------------------------------------ */
/* IEEE binary16 <-> binary32 (round-to-nearest-even), the semantics of      */
/* __half2float / __float2half in the reference kernels.             */
/* ------------------------------------------------------------------------ */

static uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

float orc_f16_to_f32(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  const uint32_t exp = (h >> 10) & 0x1Fu;
  const uint32_t man = h & 0x3FFu;
  if (exp == 0) {
    /* zero or subnormal: man * 2^-24, exact in fp32 */
    float v = (float)man * u2f(0x33800000u); /* 2^-24 */
    return u2f(f2u(v) | sign);
  }
  if (exp == 31) return u2f(sign | 0x7F800000u | (man << 13));
  return u2f(sign | ((exp + 112u) << 23) | (man << 13));
}

uint16_t orc_f32_to_f16(float f) {
  const uint32_t u = f2u(f);
  const uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
  const uint32_t a = u & 0x7FFFFFFFu;
  if (a > 0x7F800000u) return (uint16_t)(sign | 0x7E00u | ((a >> 13) & 0x3FFu)); /* NaN */
  if (a >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u); /* rounds to >= 65520 -> inf */
  if (a < 0x38800000u) {
    /* result is subnormal (or zero): units of 2^-24, round half to even */
    if (a < 0x33000000u) return sign; /* < 2^-25: rounds to 0 (2^-25 tie -> even 0) */
    const uint32_t e = a >> 23;            /* biased exponent, 102..112 */
    const uint32_t m = (a & 0x7FFFFFu) | 0x800000u;
    const uint32_t shift = 126u - e;       /* value = m * 2^(e-150); want units 2^-24 */
    uint32_t q = m >> shift;
    const uint32_t rem = m & ((1u << shift) - 1u);
    const uint32_t half = 1u << (shift - 1u);
    if (rem > half || (rem == half && (q & 1u))) ++q;
    return (uint16_t)(sign | q);
  }
  /* normal: rebias exponent, round mantissa 23 -> 10 bits */
  uint32_t v = a - 0x38000000u; /* exponent -= 112 */
  const uint32_t rem = v & 0x1FFFu;
  v >>= 13;
  if (rem > 0x1000u || (rem == 0x1000u && (v & 1u))) ++v; /* carry may bump exp: correct */
  return (uint16_t)(sign | v);
}

static uint16_t rd16(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }
static void wr16(uint8_t *p, uint16_t v) { p[0] = (uint8_t)v; p[1] = (uint8_t)(v >> 8); }

/* ------------------------------------------------------------------------ */
/* Q4_K 6-bit scale/min unpack: native/kernels/quant_common.cuh:83-94        */
/* ------------------------------------------------------------------------ */
void orc_get_scale_min_k4(int j, const uint8_t *q, uint8_t *d, uint8_t *m) {
  if (j < 4) {
    *d = q[j] & 63;
    *m = q[j + 4] & 63;
  } else {
    *d = (uint8_t)((q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4));
    *m = (uint8_t)((q[j + 4] >> 4) | ((q[j] >> 6) << 4));
  }
}

/* ------------------------------------------------------------------------ */
/* Element dequantization (fp32, no contraction)                             */
/* ------------------------------------------------------------------------ */

/* native/kernels/quant_common.cuh:100-112:
 *   w = d*sc*q - dmin*m, q = nibble of qs[(sb/2)*32 + e] (low when sb even).
 * Evaluated left to right in fp32: ((d*sc)*q) - (dmin*m).                  */
static void dequant_q4_k_block(const uint8_t *b, float *out) {
  const float d = orc_f16_to_f32(rd16(b));
  const float dmin = orc_f16_to_f32(rd16(b + 2));
  const uint8_t *scales = b + 4;
  const uint8_t *qs = b + 16;
  for (int sb = 0; sb < 8; ++sb) {
    uint8_t sc, m;
    orc_get_scale_min_k4(sb, scales, &sc, &m);
    for (int e = 0; e < 32; ++e) {
      const uint8_t qb = qs[(sb / 2) * 32 + e];
      const int q = (sb & 1) ? (qb >> 4) : (qb & 0x0F);
      out[sb * 32 + e] = d * (float)sc * (float)q - dmin * (float)m;
    }
  }
}

/* native/kernels/quant_common.cuh:161-177 (layout dequantization.cuh:41-49):
 *   q = (ql nibble | qh 2 bits << 4) - 32; w = d*scale*q.                   */
static void dequant_q6_k_block(const uint8_t *b, float *out) {
  const uint8_t *ql = b;
  const uint8_t *qh = b + 128;
  const int8_t *scales = (const int8_t *)(b + 192);
  const float d = orc_f16_to_f32(rd16(b + 208));
  for (int g = 0; g < 2; ++g)
    for (int sub = 0; sub < 4; ++sub)
      for (int e = 0; e < 32; ++e) {
        const uint8_t lb = ql[g * 64 + ((sub & 1) ? 32 : 0) + e];
        const int lv = (sub >= 2) ? (lb >> 4) : (lb & 0x0F);
        const int hv = (qh[g * 32 + e] >> (sub * 2)) & 0x03;
        const int q = (lv | (hv << 4)) - 32;
        const float sc = (float)scales[g * 8 + sub * 2 + e / 16];
        out[g * 128 + sub * 32 + e] = d * sc * (float)q;
      }
}

/* native/kernels/quant_common.cuh:114-143 (layout dequantization.cuh:27-37):
 *   q = nibble of qs[(sb/2)*32 + e] (low when sb even) + 16 * bit sb of
 *   qh[e]; w = d*sc*q - dmin*m, evaluated as ((d*sc)*q) - (dmin*m).         */
static void dequant_q5_k_block(const uint8_t *b, float *out) {
  const float d = orc_f16_to_f32(rd16(b));
  const float dmin = orc_f16_to_f32(rd16(b + 2));
  const uint8_t *scales = b + 4, *qh = b + 16, *qs = b + 48;
  for (int sb = 0; sb < 8; ++sb) {
    uint8_t sc, m;
    orc_get_scale_min_k4(sb, scales, &sc, &m);
    for (int e = 0; e < 32; ++e) {
      const uint8_t qb = qs[(sb / 2) * 32 + e];
      const int q = ((sb & 1) ? (qb >> 4) : (qb & 0x0F)) + (((qh[e] >> sb) & 1) ? 16 : 0);
      out[sb * 32 + e] = d * (float)sc * (float)q - dmin * (float)m;
    }
  }
}

/* native/kernels/quant_common.cuh:196-199 (layout dequantization.cuh:165-176):
 *   w = d*q with an fp32 d.                                                 */
static void dequant_q8_k_block(const uint8_t *b, float *out) {
  float d;
  memcpy(&d, b, 4);
  const int8_t *qs = (const int8_t *)(b + 4);
  for (int e = 0; e < 256; ++e) out[e] = d * (float)qs[e];
}

/* native/kernels/quant_common.cuh:185-188: w = d*q */
static void dequant_q8_0_block(const uint8_t *b, float *out) {
  const float d = orc_f16_to_f32(rd16(b));
  const int8_t *qs = (const int8_t *)(b + 2);
  for (int e = 0; e < 32; ++e) out[e] = d * (float)qs[e];
}

/* Whole-tensor dequant to fp32 (the reference's dequantize_{q4_k,q6_k,q8_0}
 * kernels, native/kernels/dequantization.cu:14-141, emit fp16 of the same
 * fp32 value).  W is [n_rows][K/QK] blocks, out is [n_rows][K].  Returns 0 on
 * success, 1 for an unsupported type or K.                                  */
int orc_dequantize(int qtype, const void *w, float *out, int64_t n_rows, int64_t K) {
  const int qk = orc_block_elems(qtype), bb = orc_block_bytes(qtype);
  if (!qk || qtype == ORC_Q8_1 || K % qk) return 1;
  const uint8_t *p = (const uint8_t *)w;
  const int64_t nb = n_rows * (K / qk);
  for (int64_t i = 0; i < nb; ++i) {
    const uint8_t *b = p + i * bb;
    float *o = out + i * qk;
    if (qtype == ORC_Q4_K) dequant_q4_k_block(b, o);
    else if (qtype == ORC_Q5_K) dequant_q5_k_block(b, o);
    else if (qtype == ORC_Q6_K) dequant_q6_k_block(b, o);
    else if (qtype == ORC_Q8_K) dequant_q8_k_block(b, o);
    else dequant_q8_0_block(b, o);
  }
  return 0;
}

/* ------------------------------------------------------------------------ */
/* Q8_1 activation quantizer: native/kernels/fused_dequant_gemv.cuh:597-655  */
/*   per 32: amax = max|x|; d = amax/127; inv = amax>0 ? 127/amax : 0;        */
/*   q = clamp(rint(x*inv), -128, 127); ds = {f16(d), f16(d*sum(q))}.         */
/* The reference reads fp16 input; the fp32 entry point is the BASELINE       */
/* contract.  rintf rounds half to even (the default rounding mode), as       */
/* __float2int_rn does.                                                      */
/* ------------------------------------------------------------------------ */
static void quantize_q8_1_block(const float *x, uint8_t *out) {
  float amax = 0.0f;
  for (int i = 0; i < 32; ++i) {
    const float a = fabsf(x[i]);
    amax = a > amax ? a : amax;
  }
  const float d = amax / 127.0f;
  const float inv = (amax > 0.0f) ? 127.0f / amax : 0.0f;
  int sum = 0;
  for (int i = 0; i < 32; ++i) {
    const float v = x[i] * inv;
    int q = (int)rintf(v);
    q = q < -128 ? -128 : (q > 127 ? 127 : q);
    out[4 + i] = (uint8_t)(int8_t)q;
    sum += q;
  }
  wr16(out, orc_f32_to_f16(d));
  wr16(out + 2, orc_f32_to_f16(d * (float)sum));
}

int orc_quantize_q8_1_f32(const float *x, void *out, int64_t M, int64_t K) {
  if (K % 32) return 1;
  uint8_t *o = (uint8_t *)out;
  for (int64_t i = 0; i < M * (K / 32); ++i) quantize_q8_1_block(x + i * 32, o + i * 36);
  return 0;
}

int orc_quantize_q8_1_f16(const uint16_t *x, void *out, int64_t M, int64_t K) {
  if (K % 32) return 1;
  uint8_t *o = (uint8_t *)out;
  float tmp[32];
  for (int64_t i = 0; i < M * (K / 32); ++i) {
    for (int e = 0; e < 32; ++e) tmp[e] = orc_f16_to_f32(x[i * 32 + e]);
    quantize_q8_1_block(tmp, o + i * 36);
  }
  return 0;
}

/* ------------------------------------------------------------------------ */
/* Fused producers of Q8_1 activations.                                      */
/* RMSNorm + Q8_1: native/kernels/fused_dequant_gemv.cuh:736-904 (and the    */
/*   helpers LoadHalfToSmemSumSq / ApplyNormInPlace, :24-63): per row,       */
/*   rms = rsqrt(sum(x^2)/K + eps), y = (x * rms) * w, then the quantizer.   */
/*   Here rms is evaluated in fp64 and rounded once to fp32 (the device     */
/*   result differs by rounding only), y in fp32 as two rounded products.   */
/* SiLU*mul + Q8_1: fused_dequant_gemv.cuh:657-734: y = (g / (1 + exp(-g)))  */
/*   * u; the silu factor in fp64 rounded to fp32, the product in fp32.     */
/* The *_values functions return y (the pre-quantization fp32 values).      */
/* ------------------------------------------------------------------------ */
static float rms_factor(const float *x, int64_t K, float eps) {
  double ss = 0.0;
  for (int64_t i = 0; i < K; ++i) ss += (double)x[i] * (double)x[i];
  return (float)(1.0 / sqrt(ss / (double)K + (double)eps));
}

int orc_rmsnorm_values(const float *x, const uint16_t *w, float *y, int64_t M, int64_t K,
                       float eps) {
  if (K % 32) return 1;
  for (int64_t m = 0; m < M; ++m) {
    const float *xr = x + m * K;
    const float rms = rms_factor(xr, K, eps);
    for (int64_t i = 0; i < K; ++i) {
      const float t = xr[i] * rms;
      y[m * K + i] = t * orc_f16_to_f32(w[i]);
    }
  }
  return 0;
}

int orc_rmsnorm_quantize_q8_1(const float *x, const uint16_t *w, void *out, int64_t M, int64_t K,
                              float eps) {
  if (K % 32) return 1;
  float *y = (float *)malloc(sizeof(float) * (size_t)K);
  if (!y) return 2;
  uint8_t *o = (uint8_t *)out;
  for (int64_t m = 0; m < M; ++m) {
    orc_rmsnorm_values(x + m * K, w, y, 1, K, eps);
    for (int64_t b = 0; b < K / 32; ++b) quantize_q8_1_block(y + b * 32, o + (m * (K / 32) + b) * 36);
  }
  free(y);
  return 0;
}

int orc_silu_mul_values(const float *g, const float *u, float *y, int64_t n) {
  for (int64_t i = 0; i < n; ++i) {
    const float s = (float)((double)g[i] / (1.0 + exp(-(double)g[i])));
    y[i] = s * u[i];
  }
  return 0;
}

int orc_silu_mul_quantize_q8_1(const float *g, const float *u, void *out, int64_t M, int64_t K) {
  if (K % 32) return 1;
  float y[32];
  uint8_t *o = (uint8_t *)out;
  for (int64_t b = 0; b < M * (K / 32); ++b) {
    orc_silu_mul_values(g + b * 32, u + b * 32, y, 32);
    quantize_q8_1_block(y, o + b * 36);
  }
  return 0;
}

/* ------------------------------------------------------------------------ */
/* Exact GEMV/GEMM in fp64 (the mathematical target).                        */
/*   y[m][n] = sum_k w[n][k] * a[m][k], w the exact dequantized weight        */
/*   (each w is exact in fp64) and a = f16(d_blk) * q (exact in fp64).        */
/* Same construction as the reference's host check                            */
/* (tests/unit/test_native_forward.cpp:4690-4721) but in fp64 and without     */
/* rounding W to fp16.                                                        */
/* ------------------------------------------------------------------------ */
static void dequant_row_f64(int qtype, const uint8_t *row, double *out, int64_t K) {
  const int qk = orc_block_elems(qtype), bb = orc_block_bytes(qtype);
  for (int64_t blk = 0; blk < K / qk; ++blk) {
    const uint8_t *b = row + blk * bb;
    double *o = out + blk * qk;
    if (qtype == ORC_Q4_K) {
      const double d = orc_f16_to_f32(rd16(b)), dmin = orc_f16_to_f32(rd16(b + 2));
      for (int sb = 0; sb < 8; ++sb) {
        uint8_t sc, m;
        orc_get_scale_min_k4(sb, b + 4, &sc, &m);
        for (int e = 0; e < 32; ++e) {
          const uint8_t qb = b[16 + (sb / 2) * 32 + e];
          const int q = (sb & 1) ? (qb >> 4) : (qb & 0x0F);
          o[sb * 32 + e] = d * sc * q - dmin * m;
        }
      }
    } else if (qtype == ORC_Q5_K) {
      const double d = orc_f16_to_f32(rd16(b)), dmin = orc_f16_to_f32(rd16(b + 2));
      for (int sb = 0; sb < 8; ++sb) {
        uint8_t sc, m;
        orc_get_scale_min_k4(sb, b + 4, &sc, &m);
        for (int e = 0; e < 32; ++e) {
          const uint8_t qb = b[48 + (sb / 2) * 32 + e];
          const int q = ((sb & 1) ? (qb >> 4) : (qb & 0x0F)) + 16 * ((b[16 + e] >> sb) & 1);
          o[sb * 32 + e] = d * sc * q - dmin * m;
        }
      }
    } else if (qtype == ORC_Q6_K) {
      const double d = orc_f16_to_f32(rd16(b + 208));
      for (int g = 0; g < 2; ++g)
        for (int sub = 0; sub < 4; ++sub)
          for (int e = 0; e < 32; ++e) {
            const uint8_t lb = b[g * 64 + ((sub & 1) ? 32 : 0) + e];
            const int lv = (sub >= 2) ? (lb >> 4) : (lb & 0x0F);
            const int hv = (b[128 + g * 32 + e] >> (sub * 2)) & 3;
            const int sc = ((const int8_t *)(b + 192))[g * 8 + sub * 2 + e / 16];
            o[g * 128 + sub * 32 + e] = d * sc * ((lv | (hv << 4)) - 32);
          }
    } else if (qtype == ORC_Q8_K) {
      float df;
      memcpy(&df, b, 4);
      for (int e = 0; e < 256; ++e) o[e] = (double)df * ((const int8_t *)(b + 4))[e];
    } else {
      const double d = orc_f16_to_f32(rd16(b));
      for (int e = 0; e < 32; ++e) o[e] = d * ((const int8_t *)(b + 2))[e];
    }
  }
}

static void act_row_f64(const uint8_t *a, double *out, int64_t K) {
  for (int64_t blk = 0; blk < K / 32; ++blk) {
    const uint8_t *b = a + blk * 36;
    const double d = orc_f16_to_f32(rd16(b));
    for (int e = 0; e < 32; ++e) out[blk * 32 + e] = d * ((const int8_t *)(b + 4))[e];
  }
}

typedef struct {
  int qtype, M, N, K, t, nt;
  const uint8_t *W, *A;
  double *y;
  float *yf;
} orc_job;

static void *gemv_exact_worker(void *arg) {
  orc_job *j = (orc_job *)arg;
  const int64_t row_bytes = (int64_t)j->K / orc_block_elems(j->qtype) * orc_block_bytes(j->qtype);
  double *w = (double *)malloc(sizeof(double) * j->K);
  double *a = (double *)malloc(sizeof(double) * (size_t)j->K * j->M);
  for (int m = 0; m < j->M; ++m) act_row_f64(j->A + (int64_t)m * (j->K / 32) * 36, a + (int64_t)m * j->K, j->K);
  for (int n = j->t; n < j->N; n += j->nt) {
    dequant_row_f64(j->qtype, j->W + n * row_bytes, w, j->K);
    for (int m = 0; m < j->M; ++m) {
      const double *am = a + (int64_t)m * j->K;
      double s = 0.0;
      for (int k = 0; k < j->K; ++k) s += w[k] * am[k];
      j->y[(int64_t)m * j->N + n] = s;
    }
  }
  free(w);
  free(a);
  return NULL;
}

static int check_geom(int qtype, int M, int N, int K) {
  if (qtype != ORC_Q4_K && qtype != ORC_Q5_K && qtype != ORC_Q6_K && qtype != ORC_Q8_0 &&
      qtype != ORC_Q8_K)
    return 1;
  if (M <= 0 || N <= 0 || K <= 0 || K % orc_block_elems(qtype)) return 1;
  return 0;
}

static void run_jobs(orc_job *tmpl, int threads, void *(*fn)(void *)) {
  if (threads < 1) threads = 1;
  if (threads > 256) threads = 256;
  pthread_t th[256];
  orc_job jobs[256];
  for (int t = 0; t < threads; ++t) {
    jobs[t] = *tmpl;
    jobs[t].t = t;
    jobs[t].nt = threads;
    pthread_create(&th[t], NULL, fn, &jobs[t]);
  }
  for (int t = 0; t < threads; ++t) pthread_join(th[t], NULL);
}

/* y is [M][N] fp64.  A is Q8_1 [M][K/32]. */
int orc_gemv_exact(int qtype, const void *W, const void *A, double *y, int M, int N, int K, int threads) {
  if (check_geom(qtype, M, N, K)) return 1;
  orc_job job = {qtype, M, N, K, 0, 1, (const uint8_t *)W, (const uint8_t *)A, y, NULL};
  run_jobs(&job, threads, gemv_exact_worker);
  return 0;
}

/* ------------------------------------------------------------------------ */
/* Packed (per-row symmetric int8) activations.                               */
/* Quantizer: native/cuda_kernels.cu:309-369 (QuantizeRowsSymmetricKernel):   */
/*   amax = max|x| over the row; scale = amax > 0 ? amax / 127 : 0;           */
/*   inv = scale > 0 ? 1 / scale : 0; q = clamp(rint(x * inv), -127, 127),    */
/*   all in fp32; SiLU form (:371-437) on y = silu(g) * u as                  */
/*   orc_silu_mul_values computes it.                                         */
/* GEMV: native/kernels/fused_dequant_gemv.cuh:80-580 (the *_dp4a_packed      */
/*   kernels): y[m][n] = scale[m] * sum_k w[n][k] * q[m][k], here in fp64     */
/*   from the exact dequantized row (dequant_row_f64) and the exact codes.    */
/* ------------------------------------------------------------------------ */
static void quantize_row_sym(const float *y, int8_t *codes, float *scale, int64_t K) {
  float amax = 0.0f;
  for (int64_t i = 0; i < K; ++i) amax = fmaxf(amax, fabsf(y[i]));
  const float sc = amax > 0.0f ? amax / 127.0f : 0.0f;
  const float inv = sc > 0.0f ? 1.0f / sc : 0.0f;
  *scale = sc;
  for (int64_t i = 0; i < K; ++i) {
    const float t = y[i] * inv;
    float q = rintf(t);
    if (q > 127.0f) q = 127.0f;
    if (q < -127.0f) q = -127.0f;
    codes[i] = (int8_t)q;
  }
}

int orc_quantize_rows_symmetric(const float *x, int8_t *codes, float *scales, int64_t M, int64_t K) {
  if (M < 0 || K <= 0) return 1;
  for (int64_t m = 0; m < M; ++m) quantize_row_sym(x + m * K, codes + m * K, scales + m, K);
  return 0;
}

int orc_silu_mul_quantize_rows_symmetric(const float *g, const float *u, int8_t *codes,
                                         float *scales, int64_t M, int64_t K) {
  if (M < 0 || K <= 0) return 1;
  float *y = (float *)malloc(sizeof(float) * (size_t)K);
  if (!y) return 2;
  for (int64_t m = 0; m < M; ++m) {
    orc_silu_mul_values(g + m * K, u + m * K, y, K);
    quantize_row_sym(y, codes + m * K, scales + m, K);
  }
  free(y);
  return 0;
}

typedef struct {
  int qtype, M, N, K, t, nt;
  const uint8_t *W;
  const int8_t *X;
  const float *scales;
  double *y;
} orc_packed_job;

static void *gemv_packed_worker(void *arg) {
  orc_packed_job *j = (orc_packed_job *)arg;
  const int64_t row_bytes = (int64_t)j->K / orc_block_elems(j->qtype) * orc_block_bytes(j->qtype);
  double *w = (double *)malloc(sizeof(double) * j->K);
  for (int n = j->t; n < j->N; n += j->nt) {
    dequant_row_f64(j->qtype, j->W + n * row_bytes, w, j->K);
    for (int m = 0; m < j->M; ++m) {
      const int8_t *xm = j->X + (int64_t)m * j->K;
      double s = 0.0;
      for (int k = 0; k < j->K; ++k) s += w[k] * xm[k];
      j->y[(int64_t)m * j->N + n] = s * (double)j->scales[m];
    }
  }
  free(w);
  return NULL;
}

/* y is [M][N] fp64; codes [M][K] int8; scales [M] fp32. */
int orc_gemv_packed_exact(int qtype, const void *W, const int8_t *codes, const float *scales,
                          double *y, int M, int N, int K, int threads) {
  if (check_geom(qtype, M, N, K)) return 1;
  if (threads < 1) threads = 1;
  if (threads > 256) threads = 256;
  pthread_t th[256];
  orc_packed_job jobs[256];
  for (int t = 0; t < threads; ++t) {
    orc_packed_job jb = {qtype, M, N, K, t, threads, (const uint8_t *)W, codes, scales, y};
    jobs[t] = jb;
    pthread_create(&th[t], NULL, gemv_packed_worker, &jobs[t]);
  }
  for (int t = 0; t < threads; ++t) pthread_join(th[t], NULL);
  return 0;
}

/* ------------------------------------------------------------------------ */
/* The reference kernels' own arithmetic, restated on the CPU in fp32:        */
/* integer dot over each 32-element (Q4_K, Q8_0) or 16-element (Q6_K)         */
/* sub-block, then fp32 scaling; the Q4_K min term uses the Q8_1 s field.     */
/*   Q4_K: native/kernels/mmvq.cuh:62-127                                     */
/*   Q6_K: native/kernels/mmvq.cuh:424-474                                    */
/*   Q8_0: native/kernels/mmvq.cuh:857-891                                    */
/*   Q8_K: native/kernels/mmvq.cuh:1019-1070 (fp32 d_w times d8 per 32)      */
/*   Q5_K: no reference kernel (the reference dequantizes Q5_K for cuBLAS); */
/*         the Q4_K scheme with the 5-bit code q = nibble + 16 * qh bit.    */
/* Accumulation order is per-row sequential (the reference reduces across     */
/* lanes); results agree with orc_gemv_exact to ~1e-6 relative.               */
/* ------------------------------------------------------------------------ */
static float row_dot_q8_1(int qtype, const uint8_t *row, const uint8_t *a, int K) {
  float acc = 0.0f;
  if (qtype == ORC_Q4_K) {
    for (int blk = 0; blk < K / 256; ++blk) {
      const uint8_t *b = row + blk * 144;
      const float d = orc_f16_to_f32(rd16(b)), dmin = orc_f16_to_f32(rd16(b + 2));
      for (int sb = 0; sb < 8; ++sb) {
        uint8_t sc, m;
        orc_get_scale_min_k4(sb, b + 4, &sc, &m);
        const uint8_t *ab = a + (blk * 8 + sb) * 36;
        int dot = 0;
        for (int e = 0; e < 32; ++e) {
          const uint8_t qb = b[16 + (sb / 2) * 32 + e];
          const int q = (sb & 1) ? (qb >> 4) : (qb & 0x0F);
          dot += q * (int8_t)ab[4 + e];
        }
        const float d8 = orc_f16_to_f32(rd16(ab)), s8 = orc_f16_to_f32(rd16(ab + 2));
        acc += d * (float)sc * d8 * (float)dot;
        acc -= dmin * (float)m * s8;
      }
    }
  } else if (qtype == ORC_Q5_K) {
    for (int blk = 0; blk < K / 256; ++blk) {
      const uint8_t *b = row + blk * 176;
      const float d = orc_f16_to_f32(rd16(b)), dmin = orc_f16_to_f32(rd16(b + 2));
      for (int sb = 0; sb < 8; ++sb) {
        uint8_t sc, m;
        orc_get_scale_min_k4(sb, b + 4, &sc, &m);
        const uint8_t *ab = a + (blk * 8 + sb) * 36;
        int dot = 0;
        for (int e = 0; e < 32; ++e) {
          const uint8_t qb = b[48 + (sb / 2) * 32 + e];
          const int q = ((sb & 1) ? (qb >> 4) : (qb & 0x0F)) + 16 * ((b[16 + e] >> sb) & 1);
          dot += q * (int8_t)ab[4 + e];
        }
        const float d8 = orc_f16_to_f32(rd16(ab)), s8 = orc_f16_to_f32(rd16(ab + 2));
        acc += d * (float)sc * d8 * (float)dot;
        acc -= dmin * (float)m * s8;
      }
    }
  } else if (qtype == ORC_Q8_K) {
    for (int blk = 0; blk < K / 256; ++blk) {
      const uint8_t *b = row + blk * 292;
      float dw;
      memcpy(&dw, b, 4);
      for (int sub = 0; sub < 8; ++sub) {
        const uint8_t *ab = a + (blk * 8 + sub) * 36;
        int dot = 0;
        for (int e = 0; e < 32; ++e) dot += (int8_t)b[4 + sub * 32 + e] * (int8_t)ab[4 + e];
        acc += dw * orc_f16_to_f32(rd16(ab)) * (float)dot;
      }
    }
  } else if (qtype == ORC_Q6_K) {
    for (int blk = 0; blk < K / 256; ++blk) {
      const uint8_t *b = row + blk * 210;
      const float d = orc_f16_to_f32(rd16(b + 208));
      for (int g = 0; g < 2; ++g)
        for (int sub = 0; sub < 4; ++sub) {
          const uint8_t *ab = a + (blk * 8 + g * 4 + sub) * 36;
          const float d8 = orc_f16_to_f32(rd16(ab));
          for (int h = 0; h < 2; ++h) {
            int dot = 0;
            for (int e = h * 16; e < h * 16 + 16; ++e) {
              const uint8_t lb = b[g * 64 + ((sub & 1) ? 32 : 0) + e];
              const int lv = (sub >= 2) ? (lb >> 4) : (lb & 0x0F);
              const int hv = (b[128 + g * 32 + e] >> (sub * 2)) & 3;
              dot += ((lv | (hv << 4)) - 32) * (int8_t)ab[4 + e];
            }
            const float sc = (float)((const int8_t *)(b + 192))[g * 8 + sub * 2 + h];
            acc += d * (sc * d8 * (float)dot);
          }
        }
    }
  } else {
    for (int blk = 0; blk < K / 32; ++blk) {
      const uint8_t *b = row + blk * 34;
      const uint8_t *ab = a + blk * 36;
      int dot = 0;
      for (int e = 0; e < 32; ++e) dot += (int8_t)b[2 + e] * (int8_t)ab[4 + e];
      acc += orc_f16_to_f32(rd16(b)) * orc_f16_to_f32(rd16(ab)) * (float)dot;
    }
  }
  return acc;
}

static void *gemv_q8_1_worker(void *arg) {
  orc_job *j = (orc_job *)arg;
  const int64_t row_bytes = (int64_t)j->K / orc_block_elems(j->qtype) * orc_block_bytes(j->qtype);
  for (int n = j->t; n < j->N; n += j->nt)
    for (int m = 0; m < j->M; ++m)
      j->yf[(int64_t)m * j->N + n] =
          row_dot_q8_1(j->qtype, j->W + n * row_bytes, j->A + (int64_t)m * (j->K / 32) * 36, j->K);
  return NULL;
}

int orc_gemv_q8_1(int qtype, const void *W, const void *A, float *y, int M, int N, int K, int threads) {
  if (check_geom(qtype, M, N, K)) return 1;
  orc_job job = {qtype, M, N, K, 0, 1, (const uint8_t *)W, (const uint8_t *)A, NULL, y};
  run_jobs(&job, threads, gemv_q8_1_worker);
  return 0;
}

/* ------------------------------------------------------------------------ */
/* ggml-semantics CPU baseline.                                              */
/* The reference's CPU path is ggml's vec_dot_q4_K_q8_K / vec_dot_q6_K_q8_K / */
/* vec_dot_q8_0_q8_0 inside external/llama.cpp, which is an empty submodule   */
/* in the reference snapshot (.gitmodules:1-4; called from                    */
/* runtime/backends/llama/llama_cpp_backend.cpp:543-568).  This restates the  */
/* published ggml design, not its code:                                       */
/*  - K-quants take Q8_K activations: per 256 values, fp32 d = 1/iscale with  */
/*    iscale = -127/max (max = the value of largest magnitude), q = round(x*  */
/*    iscale) clamped to 127, and int16 sums per 16 (bsums).                  */
/*  - Q8_0 weights take Q8_0 activations: per 32, d = amax/127, q = round(x/d)*/
/*  - each block: integer dot per sub-block times integer sub-block scale,    */
/*    then one fp32 scale per super-block; Q4_K mins use the bsums.           */
/* The float accumulation order of ggml's SIMD variants is not reproduced     */
/* (parity unpinned: checked only against orc_gemv_exact within tolerance).   */
/* ------------------------------------------------------------------------ */
static int nearest_int(float f) { return (int)lrintf(f); }

static void quantize_row_q8_k(const float *x, uint8_t *y, int K) {
  for (int blk = 0; blk < K / 256; ++blk) {
    const float *xb = x + blk * 256;
    uint8_t *yb = y + blk * 292;
    float amax = 0.0f, max = 0.0f;
    for (int j = 0; j < 256; ++j) {
      const float ax = fabsf(xb[j]);
      if (ax > amax) { amax = ax; max = xb[j]; }
    }
    int8_t *qs = (int8_t *)(yb + 4);
    int16_t bsums[16];
    if (amax == 0.0f) {
      float z = 0.0f;
      memcpy(yb, &z, 4);
      memset(qs, 0, 256);
      memset(bsums, 0, sizeof(bsums));
    } else {
      const float iscale = -127.0f / max;
      for (int j = 0; j < 256; ++j) {
        int v = nearest_int(iscale * xb[j]);
        qs[j] = (int8_t)(v > 127 ? 127 : (v < -128 ? -128 : v));
      }
      for (int j = 0; j < 16; ++j) {
        int s = 0;
        for (int i = 0; i < 16; ++i) s += qs[j * 16 + i];
        bsums[j] = (int16_t)s;
      }
      const float d = 1.0f / iscale;
      memcpy(yb, &d, 4);
    }
    memcpy(yb + 260, bsums, 32);
  }
}

static void quantize_row_q8_0(const float *x, uint8_t *y, int K) {
  for (int blk = 0; blk < K / 32; ++blk) {
    const float *xb = x + blk * 32;
    float amax = 0.0f;
    for (int j = 0; j < 32; ++j) { const float a = fabsf(xb[j]); if (a > amax) amax = a; }
    const float d = amax / 127.0f;
    const float id = d ? 1.0f / d : 0.0f;
    wr16(y + blk * 34, orc_f32_to_f16(d));
    for (int j = 0; j < 32; ++j) y[blk * 34 + 2 + j] = (uint8_t)(int8_t)nearest_int(xb[j] * id);
  }
}

static float vec_dot_q4_k_q8_k(const uint8_t *row, const uint8_t *q8, int K) {
  float sumf = 0.0f;
  for (int blk = 0; blk < K / 256; ++blk) {
    const uint8_t *b = row + blk * 144;
    const uint8_t *y = q8 + blk * 292;
    float dy;
    memcpy(&dy, y, 4);
    const int8_t *qy = (const int8_t *)(y + 4);
    int16_t bsums[16];
    memcpy(bsums, y + 260, 32);
    const float d = dy * orc_f16_to_f32(rd16(b));
    const float dmin = dy * orc_f16_to_f32(rd16(b + 2));
    int32_t sumi = 0, summs = 0;
    for (int sb = 0; sb < 8; ++sb) {
      uint8_t sc, m;
      orc_get_scale_min_k4(sb, b + 4, &sc, &m);
      int32_t dot = 0;
      for (int e = 0; e < 32; ++e) {
        const uint8_t qb = b[16 + (sb / 2) * 32 + e];
        dot += ((sb & 1) ? (qb >> 4) : (qb & 0xF)) * qy[sb * 32 + e];
      }
      sumi += sc * dot;
      summs += m * (bsums[2 * sb] + bsums[2 * sb + 1]);
    }
    sumf += d * (float)sumi - dmin * (float)summs;
  }
  return sumf;
}

static float vec_dot_q6_k_q8_k(const uint8_t *row, const uint8_t *q8, int K) {
  float sumf = 0.0f;
  for (int blk = 0; blk < K / 256; ++blk) {
    const uint8_t *b = row + blk * 210;
    const uint8_t *y = q8 + blk * 292;
    float dy;
    memcpy(&dy, y, 4);
    const int8_t *qy = (const int8_t *)(y + 4);
    const int8_t *sc = (const int8_t *)(b + 192);
    int32_t sumi = 0;
    for (int g = 0; g < 2; ++g)
      for (int sub = 0; sub < 4; ++sub)
        for (int h = 0; h < 2; ++h) {
          int32_t dot = 0;
          for (int e = h * 16; e < h * 16 + 16; ++e) {
            const uint8_t lb = b[g * 64 + ((sub & 1) ? 32 : 0) + e];
            const int lv = (sub >= 2) ? (lb >> 4) : (lb & 0xF);
            const int hv = (b[128 + g * 32 + e] >> (sub * 2)) & 3;
            dot += ((lv | (hv << 4)) - 32) * qy[g * 128 + sub * 32 + e];
          }
          sumi += sc[g * 8 + sub * 2 + h] * dot;
        }
    sumf += dy * orc_f16_to_f32(rd16(b + 208)) * (float)sumi;
  }
  return sumf;
}

static float vec_dot_q8_0_q8_0(const uint8_t *row, const uint8_t *q8, int K) {
  float sumf = 0.0f;
  for (int blk = 0; blk < K / 32; ++blk) {
    const uint8_t *b = row + blk * 34, *y = q8 + blk * 34;
    int32_t dot = 0;
    for (int e = 0; e < 32; ++e) dot += (int8_t)b[2 + e] * (int8_t)y[2 + e];
    sumf += orc_f16_to_f32(rd16(b)) * orc_f16_to_f32(rd16(y)) * (float)dot;
  }
  return sumf;
}

typedef struct {
  int qtype, M, N, K, t, nt;
  const uint8_t *W, *xq;
  float *y;
} ggml_job;

static void *ggml_worker(void *arg) {
  ggml_job *j = (ggml_job *)arg;
  const int64_t rb = (int64_t)j->K / orc_block_elems(j->qtype) * orc_block_bytes(j->qtype);
  const int64_t ab = j->qtype == ORC_Q8_0 ? (int64_t)j->K / 32 * 34 : (int64_t)j->K / 256 * 292;
  /* contiguous row ranges per thread */
  const int n0 = (int)((int64_t)j->N * j->t / j->nt), n1 = (int)((int64_t)j->N * (j->t + 1) / j->nt);
  for (int n = n0; n < n1; ++n)
    for (int m = 0; m < j->M; ++m) {
      const uint8_t *w = j->W + n * rb, *x = j->xq + m * ab;
      float v;
      if (j->qtype == ORC_Q4_K) v = vec_dot_q4_k_q8_k(w, x, j->K);
      else if (j->qtype == ORC_Q6_K) v = vec_dot_q6_k_q8_k(w, x, j->K);
      else v = vec_dot_q8_0_q8_0(w, x, j->K);
      j->y[(int64_t)m * j->N + n] = v;
    }
  return NULL;
}

/* x fp32 [M][K] -> y fp32 [M][N]; activation quantization is included, as in
 * ggml's mul_mat (it quantizes src1 once, then runs vec_dot per row). */
int orc_ggml_cpu_gemv(int qtype, const void *W, const float *x, float *y, int M, int N, int K, int threads) {
  if (check_geom(qtype, M, N, K)) return 1;
  if (qtype != ORC_Q8_0 && K % 256) return 1;
  const int64_t ab = qtype == ORC_Q8_0 ? (int64_t)K / 32 * 34 : (int64_t)K / 256 * 292;
  uint8_t *xq = (uint8_t *)malloc((size_t)(ab * M));
  for (int m = 0; m < M; ++m) {
    if (qtype == ORC_Q8_0) quantize_row_q8_0(x + (int64_t)m * K, xq + m * ab, K);
    else quantize_row_q8_k(x + (int64_t)m * K, xq + m * ab, K);
  }
  if (threads < 1) threads = 1;
  if (threads > 256) threads = 256;
  pthread_t th[256];
  ggml_job jobs[256];
  for (int t = 0; t < threads; ++t) {
    ggml_job jb = {qtype, M, N, K, t, threads, (const uint8_t *)W, xq, y};
    jobs[t] = jb;
    pthread_create(&th[t], NULL, ggml_worker, &jobs[t]);
  }
  for (int t = 0; t < threads; ++t) pthread_join(th[t], NULL);
  free(xq);
  return 0;
}

/* Array forms of the f16 conversions (for exhaustive checks). */
void orc_f16_to_f32_array(const uint16_t *h, float *f, int64_t n) {
  for (int64_t i = 0; i < n; ++i) f[i] = orc_f16_to_f32(h[i]);
}

void orc_f32_to_f16_array(const float *f, uint16_t *h, int64_t n) {
  for (int64_t i = 0; i < n; ++i) h[i] = orc_f32_to_f16(f[i]);
}
