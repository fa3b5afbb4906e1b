"""ctypes wrapper over the CPU oracle (oracle/liboracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, never by the inferflux_amd product package.
The arithmetic lives in ifx_oracle.c, which cites the reference lines it
restates.
"""
import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")

Q8_0, Q8_1, Q4_K, Q5_K, Q6_K, Q8_K = 8, 9, 12, 13, 14, 15
BLOCK_BYTES = {Q4_K: 144, Q5_K: 176, Q6_K: 210, Q8_0: 34, Q8_1: 36, Q8_K: 292}
BLOCK_ELEMS = {Q4_K: 256, Q5_K: 256, Q6_K: 256, Q8_0: 32, Q8_1: 32, Q8_K: 256}

_lib = None


def build(force=False):
    """Compile liboracle.so with the committed Makefile."""
    if force or not os.path.exists(LIB_PATH):
        subprocess.run(["make", "-s", "-C", HERE] + (["-B"] if force else []), check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = ctypes.CDLL(LIB_PATH)
        vp, i64, i32 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int
        L.orc_f16_to_f32.argtypes = [ctypes.c_uint16]
        L.orc_f16_to_f32.restype = ctypes.c_float
        L.orc_f32_to_f16.argtypes = [ctypes.c_float]
        L.orc_f32_to_f16.restype = ctypes.c_uint16
        L.orc_f16_to_f32_array.argtypes = [vp, vp, i64]
        L.orc_f32_to_f16_array.argtypes = [vp, vp, i64]
        L.orc_get_scale_min_k4.argtypes = [i32, vp, vp, vp]
        L.orc_dequantize.argtypes = [i32, vp, vp, i64, i64]
        L.orc_quantize_q8_1_f32.argtypes = [vp, vp, i64, i64]
        L.orc_quantize_q8_1_f16.argtypes = [vp, vp, i64, i64]
        L.orc_rmsnorm_values.argtypes = [vp, vp, vp, i64, i64, ctypes.c_float]
        L.orc_rmsnorm_quantize_q8_1.argtypes = [vp, vp, vp, i64, i64, ctypes.c_float]
        L.orc_silu_mul_values.argtypes = [vp, vp, vp, i64]
        L.orc_silu_mul_quantize_q8_1.argtypes = [vp, vp, vp, i64, i64]
        L.orc_gemv_exact.argtypes = [i32, vp, vp, vp, i32, i32, i32, i32]
        L.orc_gemv_q8_1.argtypes = [i32, vp, vp, vp, i32, i32, i32, i32]
        L.orc_ggml_cpu_gemv.argtypes = [i32, vp, vp, vp, i32, i32, i32, i32]
        L.orc_quantize_rows_symmetric.argtypes = [vp, vp, vp, i64, i64]
        L.orc_silu_mul_quantize_rows_symmetric.argtypes = [vp, vp, vp, vp, i64, i64]
        L.orc_gemv_packed_exact.argtypes = [i32, vp, vp, vp, vp, i32, i32, i32, i32]
        _lib = L
    return _lib


def _p(a):
    return ctypes.c_void_p(a.ctypes.data)


def _threads(threads):
    return threads if threads else min(os.cpu_count() or 1, 64)


def f16_to_f32(h):
    return lib().orc_f16_to_f32(int(h))


def f32_to_f16(f):
    return lib().orc_f32_to_f16(float(f))


def f16_bits_to_f32(h):
    h = np.ascontiguousarray(h, dtype=np.uint16)
    out = np.empty(h.shape, np.float32)
    lib().orc_f16_to_f32_array(_p(h), _p(out), h.size)
    return out


def f32_to_f16_bits(f):
    f = np.ascontiguousarray(f, dtype=np.float32)
    out = np.empty(f.shape, np.uint16)
    lib().orc_f32_to_f16_array(_p(f), _p(out), f.size)
    return out


def get_scale_min_k4(j, scales12):
    s = np.ascontiguousarray(scales12, dtype=np.uint8)
    d = np.zeros(1, np.uint8)
    m = np.zeros(1, np.uint8)
    lib().orc_get_scale_min_k4(j, _p(s), _p(d), _p(m))
    return int(d[0]), int(m[0])


def dequantize(qtype, w_bytes, n_rows, K):
    w = np.ascontiguousarray(w_bytes, dtype=np.uint8)
    out = np.empty((n_rows, K), np.float32)
    rc = lib().orc_dequantize(qtype, _p(w), _p(out), n_rows, K)
    if rc:
        raise ValueError("orc_dequantize: unsupported type/K")
    return out


def quantize_q8_1(x):
    """x: [M][K] float32 or float16 -> uint8 [M][K/32*36] Q8_1 blocks."""
    x = np.ascontiguousarray(x)
    M, K = x.shape
    out = np.empty((M, K // 32 * 36), np.uint8)
    if x.dtype == np.float16:
        rc = lib().orc_quantize_q8_1_f16(_p(x), _p(out), M, K)
    else:
        x = np.ascontiguousarray(x, dtype=np.float32)
        rc = lib().orc_quantize_q8_1_f32(_p(x), _p(out), M, K)
    if rc:
        raise ValueError("K must be a multiple of 32")
    return out


def _f32(x):
    """fp16 inputs are widened exactly, as the device kernels do."""
    return np.ascontiguousarray(np.asarray(x).astype(np.float32))


def rmsnorm_values(x, w_f16, eps):
    """fp32 pre-quantization values of RMSNorm: (x * rms) * w."""
    x = _f32(x)
    M, K = x.shape
    w = np.ascontiguousarray(w_f16, dtype=np.float16).view(np.uint16)
    y = np.empty_like(x)
    lib().orc_rmsnorm_values(_p(x), _p(w), _p(y), M, K, eps)
    return y


def rmsnorm_quantize_q8_1(x, w_f16, eps):
    x = _f32(x)
    M, K = x.shape
    w = np.ascontiguousarray(w_f16, dtype=np.float16).view(np.uint16)
    out = np.empty((M, K // 32 * 36), np.uint8)
    if lib().orc_rmsnorm_quantize_q8_1(_p(x), _p(w), _p(out), M, K, eps):
        raise ValueError("K must be a multiple of 32")
    return out


def silu_mul_values(g, u):
    g, u = _f32(g), _f32(u)
    y = np.empty_like(g)
    lib().orc_silu_mul_values(_p(g), _p(u), _p(y), g.size)
    return y


def silu_mul_quantize_q8_1(g, u):
    g, u = _f32(g), _f32(u)
    M, K = g.shape
    out = np.empty((M, K // 32 * 36), np.uint8)
    if lib().orc_silu_mul_quantize_q8_1(_p(g), _p(u), _p(out), M, K):
        raise ValueError("K must be a multiple of 32")
    return out


def gemv_exact(qtype, w_bytes, act_q8_1, M, N, K, threads=0):
    """fp64 y[M][N] from exact dequantized W and exact Q8_1 activations."""
    w = np.ascontiguousarray(w_bytes, dtype=np.uint8)
    a = np.ascontiguousarray(act_q8_1, dtype=np.uint8)
    y = np.empty((M, N), np.float64)
    if lib().orc_gemv_exact(qtype, _p(w), _p(a), _p(y), M, N, K, _threads(threads)):
        raise ValueError("unsupported geometry")
    return y


def gemv_q8_1(qtype, w_bytes, act_q8_1, M, N, K, threads=0):
    """fp32 y[M][N] with the reference kernels' integer-dot arithmetic."""
    w = np.ascontiguousarray(w_bytes, dtype=np.uint8)
    a = np.ascontiguousarray(act_q8_1, dtype=np.uint8)
    y = np.empty((M, N), np.float32)
    if lib().orc_gemv_q8_1(qtype, _p(w), _p(a), _p(y), M, N, K, _threads(threads)):
        raise ValueError("unsupported geometry")
    return y


def ggml_cpu_gemv(qtype, w_bytes, x, N, threads=0):
    """ggml-semantics CPU baseline: fp32 x [M][K] -> fp32 y [M][N]."""
    w = np.ascontiguousarray(w_bytes, dtype=np.uint8)
    x = np.ascontiguousarray(x, dtype=np.float32)
    M, K = x.shape
    y = np.empty((M, N), np.float32)
    if lib().orc_ggml_cpu_gemv(qtype, _p(w), _p(x), _p(y), M, N, K, _threads(threads)):
        raise ValueError("unsupported geometry")
    return y


def quantize_rows_symmetric(x):
    """(int8 codes [M][K], fp32 scales [M]) of fp32 x [M][K]."""
    x = _f32(x)
    M, K = x.shape
    codes = np.empty((M, K), np.int8)
    scales = np.empty(M, np.float32)
    if lib().orc_quantize_rows_symmetric(_p(x), _p(codes), _p(scales), M, K):
        raise ValueError("bad shape")
    return codes, scales


def silu_mul_quantize_rows_symmetric(g, u):
    g, u = _f32(g), _f32(u)
    M, K = g.shape
    codes = np.empty((M, K), np.int8)
    scales = np.empty(M, np.float32)
    if lib().orc_silu_mul_quantize_rows_symmetric(_p(g), _p(u), _p(codes), _p(scales), M, K):
        raise ValueError("bad shape")
    return codes, scales


def gemv_packed_exact(qtype, w_bytes, codes, scales, M, N, K, threads=0):
    """fp64 y[M][N] = scale[m] * (exact dequantized W . int8 codes)."""
    w = np.ascontiguousarray(w_bytes, dtype=np.uint8)
    c = np.ascontiguousarray(codes, dtype=np.int8)
    s = np.ascontiguousarray(scales, dtype=np.float32)
    y = np.empty((M, N), np.float64)
    if lib().orc_gemv_packed_exact(qtype, _p(w), _p(c), _p(s), _p(y), M, N, K, _threads(threads)):
        raise ValueError("unsupported geometry")
    return y


def row_norm_tolerance(y_ref, rel=1e-3):
    """Per output row m: allowed max |err| = rel * ||y_ref[m, :]||_2."""
    return rel * np.linalg.norm(np.asarray(y_ref, np.float64), axis=1)
