"""Seeded synthetic GGUF blocks and activations for the benchmark configs.

numpy's PCG64 generator (np.random.default_rng(seed)) produces the bytes on
the host; the same bytes are uploaded to the GPU and handed to the CPU
checker, so both sides see identical inputs.  Distributions follow the
benchmark configs:
  Q4_K  d, dmin = f16(|N(0,1)| * 0.01); 12 scale bytes and 128 qs bytes
        uniform (uniform bytes give uniform 6-bit scales/mins and nibbles)
  Q6_K  ql, qh bytes uniform; scales int8 uniform in [-64, 63];
        d = f16(|N(0,1)| * 0.01)                       (d is the LAST field)
  Q8_0  d = f16(|N(0,1)| * 0.01); qs int8 uniform in [-127, 127]
  Q5_K  as Q4_K, plus 32 qh bytes uniform
  Q8_K  d = fp32 |N(0,1)| * 0.01; qs int8 uniform in [-127, 127]; bsums the
        int16 sums of each 16 codes (as ggml's quantize_row_q8_K stores them)
  x     N(0,1) fp32, optionally with a seeded 1% of the K channels x20
"""
import numpy as np

from .ops import Q4_K, Q5_K, Q6_K, Q8_0, Q8_K, BLOCK_BYTES, BLOCK_ELEMS


def _f16_abs_normal(rng, n, scale=0.01):
    return (np.abs(rng.standard_normal(n)) * scale).astype(np.float16).view(np.uint8).reshape(n, 2)


def blocks(qtype, n_rows, K, seed):
    """uint8 [n_rows, K/QK*bytes] raw GGUF blocks."""
    nb = n_rows * (K // BLOCK_ELEMS[qtype])
    rng = np.random.default_rng(seed)
    out = np.empty((nb, BLOCK_BYTES[qtype]), np.uint8)
    if qtype == Q4_K:
        out[:, 0:2] = _f16_abs_normal(rng, nb)
        out[:, 2:4] = _f16_abs_normal(rng, nb)
        out[:, 4:144] = rng.integers(0, 256, (nb, 140), dtype=np.uint8)
    elif qtype == Q6_K:
        out[:, 0:192] = rng.integers(0, 256, (nb, 192), dtype=np.uint8)
        out[:, 192:208] = rng.integers(-64, 64, (nb, 16), dtype=np.int8).view(np.uint8)
        out[:, 208:210] = _f16_abs_normal(rng, nb)
    elif qtype == Q8_0:
        out[:, 0:2] = _f16_abs_normal(rng, nb)
        out[:, 2:34] = rng.integers(-127, 128, (nb, 32), dtype=np.int8).view(np.uint8)
    elif qtype == Q5_K:
        out[:, 0:2] = _f16_abs_normal(rng, nb)
        out[:, 2:4] = _f16_abs_normal(rng, nb)
        out[:, 4:176] = rng.integers(0, 256, (nb, 172), dtype=np.uint8)
    elif qtype == Q8_K:
        out[:, 0:4] = (np.abs(rng.standard_normal(nb)) * 0.01).astype(np.float32).view(np.uint8).reshape(nb, 4)
        qs = rng.integers(-127, 128, (nb, 256), dtype=np.int8)
        out[:, 4:260] = qs.view(np.uint8)
        out[:, 260:292] = qs.reshape(nb, 16, 16).sum(axis=2, dtype=np.int16).view(np.uint8)
    else:
        raise ValueError(qtype)
    return out.reshape(n_rows, -1)


def activations(M, K, seed, outlier_frac=0.0, outlier_scale=20.0):
    """fp32 [M, K] ~ N(0,1); a seeded outlier_frac of channels scaled."""
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((M, K), dtype=np.float32)
    if outlier_frac > 0:
        n_out = max(1, int(round(K * outlier_frac)))
        ch = rng.choice(K, n_out, replace=False)
        x[:, ch] *= np.float32(outlier_scale)
    return x
