"""Pins the CPU oracle (oracle/ifx_oracle.c) before it is trusted as the
checker: exhaustive fp16 conversion, the 6-bit scale packing, hand-built
blocks with closed-form answers, the reference's Q8_1 known-answer pattern,
and brute force against an independent numpy statement of the formats."""
import json
import os

import numpy as np
import pytest

from tests import qref

Q8_0, Q8_1, Q4_K, Q5_K, Q6_K, Q8_K = 8, 9, 12, 13, 14, 15
GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


# --------------------------------------------------------------------- fp16
def test_f16_decode_exhaustive(orc):
    codes = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = orc.f16_bits_to_f32(codes)
    want = codes.view(np.float16).astype(np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def test_f16_encode_matches_numpy_rne(orc):
    rng = np.random.default_rng(1)
    # random bit patterns over the whole float32 range, plus every float32
    # that is exactly halfway between adjacent fp16 values (ties) near 1,
    # subnormals and the overflow boundary
    bits = rng.integers(0, 2**32, 2**20, dtype=np.uint64).astype(np.uint32)
    f = bits.view(np.float32)
    h = np.arange(0x3C00, 0x3C00 + 1024, dtype=np.uint16).view(np.float16).astype(np.float32)
    ties = (h[:-1] + h[1:]) / 2
    sub = (np.arange(0, 2048, dtype=np.float32) * np.float32(2.0**-25))
    edge = np.array([65504.0, 65519.99, 65520.0, 65536.0, -65520.0, 2.0**-24, 2.0**-25,
                     3 * 2.0**-26, 6.1e-5, -0.0, 0.0, np.inf, -np.inf], np.float32)
    allf = np.concatenate([f, ties, -ties, sub, -sub, edge])
    allf = allf[~np.isnan(allf)]
    got = orc.f32_to_f16_bits(allf)
    with np.errstate(over="ignore"):
        want = allf.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, want)


# ------------------------------------------------------------ scale packing
def test_scale_min_k4_roundtrip_all_pairs(orc):
    """Every (sc, m) in 0..63 x 0..63 at every sub-block position j."""
    vals = np.arange(64)
    sc_all, m_all = np.meshgrid(vals, vals, indexing="ij")
    sc_all, m_all = sc_all.ravel(), m_all.ravel()
    rng = np.random.default_rng(2)
    for j in range(8):
        sc = rng.integers(0, 64, (sc_all.size, 8))
        m = rng.integers(0, 64, (sc_all.size, 8))
        sc[:, j], m[:, j] = sc_all, m_all
        packed = qref.pack_scale_min_k4(sc, m)
        usc, um = qref.unpack_scale_min_k4(packed)
        assert np.array_equal(usc, sc) and np.array_equal(um, m)
        for i in range(0, sc_all.size, 97):  # oracle on a spread subset
            assert orc.get_scale_min_k4(j, packed[i]) == (sc[i, j], m[i, j])


# --------------------------------------------------------- dequant (exact)
def _q4k_block(d, dmin, sc, m, q):
    b = np.zeros(144, np.uint8)
    b[0:2] = qref.enc_half(d)
    b[2:4] = qref.enc_half(dmin)
    b[4:16] = qref.pack_scale_min_k4(np.array(sc), np.array(m))
    q = np.asarray(q).reshape(8, 32)
    for p in range(4):
        b[16 + 32 * p:48 + 32 * p] = q[2 * p] | (q[2 * p + 1] << 4)
    return b


def test_dequant_q4k_closed_form(orc):
    q = np.arange(256) % 16
    # d = 1, sc = 1, dmin = 0  ->  w = q
    b = _q4k_block(1.0, 0.0, [1] * 8, [0] * 8, q)
    assert np.array_equal(orc.dequantize(Q4_K, b, 1, 256)[0], q.astype(np.float32))
    # dmin = 1, m = 1 -> w = q - 1 ; sub-block scales differ: w = sc_j * q - m_j
    sc = [1, 2, 3, 4, 63, 32, 17, 5]
    m = [0, 1, 2, 3, 63, 40, 9, 33]
    b = _q4k_block(1.0, 1.0, sc, m, q)
    want = (np.repeat(sc, 32) * q - np.repeat(m, 32)).astype(np.float32)
    assert np.array_equal(orc.dequantize(Q4_K, b, 1, 256)[0], want)
    # fp16 scales: w = d*sc*q - dmin*m exactly as fp32 arithmetic
    b = _q4k_block(0.0123, 0.0077, sc, m, q)
    d, dmin = np.float32(np.float16(0.0123)), np.float32(np.float16(0.0077))
    want = (d * np.repeat(np.float32(sc), 32) * q.astype(np.float32)
            - dmin * np.repeat(np.float32(m), 32))
    assert np.array_equal(orc.dequantize(Q4_K, b, 1, 256)[0], want)


def test_dequant_q6k_closed_form(orc):
    b = np.zeros(210, np.uint8)
    q = np.arange(256) % 64                      # element value 0..63 before -32
    for g in range(2):
        for sub in range(4):
            e = np.arange(32)
            v = q[g * 128 + sub * 32 + e]
            lo, hi = v & 0xF, v >> 4
            idx = g * 64 + (sub & 1) * 32 + e
            b[idx] |= (lo << (4 if sub >= 2 else 0)).astype(np.uint8)
            b[128 + g * 32 + e] |= (hi << (2 * sub)).astype(np.uint8)
    b[192:208] = 1
    b[208:210] = qref.enc_half(1.0)
    assert np.array_equal(orc.dequantize(Q6_K, b, 1, 256)[0], (q - 32).astype(np.float32))
    b[192:208] = np.arange(-8, 8, dtype=np.int8).view(np.uint8)
    want = (np.repeat(np.arange(-8, 8), 16) * (q - 32)).astype(np.float32)
    assert np.array_equal(orc.dequantize(Q6_K, b, 1, 256)[0], want)


def test_dequant_q8_0_closed_form(orc):
    b = np.zeros(34, np.uint8)
    b[0:2] = qref.enc_half(0.5)
    b[2:34] = np.arange(-16, 16, dtype=np.int8).view(np.uint8)
    assert np.array_equal(orc.dequantize(Q8_0, b, 1, 32)[0],
                          np.arange(-16, 16, dtype=np.float32) / 2)


def _q5k_block(d, dmin, sc, m, q):
    """q in 0..31: nibbles as Q4_K, bit 4 of value e of sub-block j in bit j of qh[e]."""
    q = np.asarray(q).reshape(8, 32)
    b4 = _q4k_block(d, dmin, sc, m, q & 0xF)
    b = np.zeros(176, np.uint8)
    b[0:16] = b4[0:16]
    b[48:176] = b4[16:144]
    for j in range(8):
        b[16:48] |= ((q[j] >> 4) << j).astype(np.uint8)
    return b


def test_dequant_q5k_closed_form(orc):
    q = np.arange(256) % 32
    b = _q5k_block(1.0, 0.0, [1] * 8, [0] * 8, q)
    assert np.array_equal(orc.dequantize(Q5_K, b, 1, 256)[0], q.astype(np.float32))
    sc = [1, 2, 3, 4, 63, 32, 17, 5]
    m = [0, 1, 2, 3, 63, 40, 9, 33]
    b = _q5k_block(1.0, 1.0, sc, m, q[::-1])
    want = (np.repeat(sc, 32) * q[::-1] - np.repeat(m, 32)).astype(np.float32)
    assert np.array_equal(orc.dequantize(Q5_K, b, 1, 256)[0], want)


def test_dequant_q5k_reduces_to_q4k(orc):
    """qh = 0: Q5_K is Q4_K on the same d, dmin, scales and qs; qh all ones
    adds 16*d*sc to every value (catches a misplaced qh bit or field)."""
    from inferflux_amd import synth
    w4 = synth.blocks(Q4_K, 3, 512, seed=21).reshape(-1, 144)
    w5 = np.zeros((w4.shape[0], 176), np.uint8)
    w5[:, 0:16], w5[:, 48:176] = w4[:, 0:16], w4[:, 16:144]
    y4 = orc.dequantize(Q4_K, w4, 3, 512).astype(np.float64)
    assert np.array_equal(orc.dequantize(Q5_K, w5, 3, 512), orc.dequantize(Q4_K, w4, 3, 512))
    w5[:, 16:48] = 0xFF
    d = qref.f16(w4[:, 0:2])
    sc, _ = qref.unpack_scale_min_k4(w4[:, 4:16])
    add = (16 * d[:, None] * sc).repeat(32, axis=1).reshape(3, 512)
    assert np.allclose(orc.dequantize(Q5_K, w5, 3, 512), y4 + add, rtol=1e-6, atol=1e-6)


def test_dequant_q8k_closed_form(orc):
    b = np.zeros(292, np.uint8)
    b[0:4] = np.array([0.25], np.float32).view(np.uint8)
    b[4:260] = np.arange(-128, 128, dtype=np.int8).view(np.uint8)
    assert np.array_equal(orc.dequantize(Q8_K, b, 1, 256)[0],
                          np.arange(-128, 128, dtype=np.float32) / 4)


@pytest.mark.parametrize("qtype", [Q4_K, Q5_K, Q6_K, Q8_0, Q8_K])
def test_dequant_matches_numpy_statement(orc, qtype):
    from inferflux_amd import synth
    K = 512
    w = synth.blocks(qtype, 7, K, seed=11)
    got = orc.dequantize(qtype, w, 7, K).astype(np.float64)
    want = qref.dequant_f64(qtype, w, 7, K)
    # fp32 rounding of d*sc*q - dmin*m vs exact float64
    assert np.allclose(got, want, rtol=2e-7, atol=1e-9)


# ---------------------------------------------------------------- Q8_1
def test_q8_1_zero_block(orc):
    a = orc.quantize_q8_1(np.zeros((1, 32), np.float32))
    assert not a.any()


def test_q8_1_one_hot_and_ties(orc):
    x = np.zeros((1, 64), np.float32)
    x[0, 5] = 3.0
    x[0, 40] = -127.0   # block 1: amax = 127 -> inv = 1.0, codes = rint(x)
    x[0, 33] = 2.5      # tie -> 2 (even)
    x[0, 34] = 3.5      # tie -> 4
    x[0, 35] = -2.5     # tie -> -2
    x[0, 36] = 0.5      # tie -> 0
    a = orc.quantize_q8_1(x)
    d, s, q = qref.q8_1_fields(a, 1, 64)
    assert q[0, 0, 5] == 127 and np.count_nonzero(q[0, 0]) == 1
    assert d[0, 0] == np.float16(np.float32(3.0) / np.float32(127.0))
    dd = np.float32(3.0) / np.float32(127.0)
    assert s[0, 0] == np.float16(dd * np.float32(127))
    assert list(q[0, 1, [8, 1, 2, 3, 4]]) == [-127, 2, 4, -2, 0]
    assert d[0, 1] == np.float16(1.0)
    assert s[0, 1] == np.float16(-127 + 2 + 4 - 2 + 0)


def test_q8_1_reference_pattern_kat(orc):
    """Values of the reference test (test_native_forward.cpp:7706-7772):
    gate = (i-16)/8, up = 1 + (i%5)/4, x = silu(gate)*up; its expected codes
    are lrint(x / (amax/127)).  The kernel formula is rint(x * (127/amax));
    the fixture records both and they agree on this pattern."""
    with open(os.path.join(GOLDEN, "q8_1_kat.json")) as f:
        kat = json.load(f)
    for case in kat["cases"]:
        x = np.array(case["x"], np.float32).reshape(1, -1)
        a = orc.quantize_q8_1(x)
        d, s, q = qref.q8_1_fields(a, 1, x.shape[1])
        assert q.ravel().tolist() == case["q"]
        assert d.view(np.uint16).ravel().tolist() == case["d_bits"]
        assert s.view(np.uint16).ravel().tolist() == case["s_bits"]
        assert case["q"] == case["q_ref_test_formula"], "kernel vs test formula differ"


def test_q8_1_properties(orc):
    rng = np.random.default_rng(3)
    x = rng.standard_normal((4, 1024)).astype(np.float32) * np.float32(3.0)
    a = orc.quantize_q8_1(x)
    d, s, q = qref.q8_1_fields(a, 4, 1024)
    xb = x.reshape(4, 32, 32)
    amax = np.abs(xb).max(axis=2)
    assert np.array_equal(d, (amax / np.float32(127)).astype(np.float16))
    # the max-magnitude element maps to +-127
    arg = np.abs(xb).argmax(axis=2)
    assert np.all(np.abs(np.take_along_axis(q, arg[..., None], 2)) == 127)
    # reconstruction error <= half a step (plus fp16 rounding of d)
    rec = d.astype(np.float32)[..., None] * q
    assert np.all(np.abs(rec - xb) <= (amax / 127 * 0.5 + amax * 1e-3)[..., None])
    # s = f16(d * sum(q)) with d in fp32
    dd = amax / np.float32(127)
    assert np.array_equal(s, (dd * q.astype(np.int32).sum(axis=2).astype(np.float32)).astype(np.float16))
    # fp16 input path equals the fp32 path on fp16-representable values
    xh = x.astype(np.float16)
    assert np.array_equal(orc.quantize_q8_1(xh), orc.quantize_q8_1(xh.astype(np.float32)))


# ------------------------------------------------------------------ GEMV
@pytest.mark.parametrize("qtype,K", [(Q4_K, 512), (Q5_K, 512), (Q6_K, 768), (Q8_0, 160),
                                     (Q8_K, 512)])
def test_gemv_exact_brute_force(orc, qtype, K):
    from inferflux_amd import synth
    M, N = 3, 9
    w = synth.blocks(qtype, N, K, seed=5)
    a = orc.quantize_q8_1(synth.activations(M, K, seed=6))
    y = orc.gemv_exact(qtype, w, a, M, N, K)
    want = qref.act_f64(a, M, K) @ qref.dequant_f64(qtype, w, N, K).T
    assert np.allclose(y, want, rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("qtype,K", [(Q4_K, 1024), (Q5_K, 1024), (Q6_K, 1024), (Q8_0, 1024),
                                     (Q8_K, 1024)])
def test_gemv_q8_1_vs_exact(orc, qtype, K):
    from inferflux_amd import synth
    M, N = 4, 64
    w = synth.blocks(qtype, N, K, seed=7)
    a = orc.quantize_q8_1(synth.activations(M, K, seed=8))
    y = orc.gemv_q8_1(qtype, w, a, M, N, K)
    ye = orc.gemv_exact(qtype, w, a, M, N, K)
    # The kernels' Q4_K min term uses the fp16-rounded s = f16(d*sum(q))
    # field (mmvq.cuh:121-125), so they differ from the exact product by
    # ~1e-5 of the row norm; the contract allows 1e-3.
    tol = orc.row_norm_tolerance(ye, 1e-4)
    assert np.all(np.abs(y - ye).max(axis=1) <= tol)


def test_gemv_linearity_and_zero(orc):
    from inferflux_amd import synth
    K, N = 512, 16
    w = synth.blocks(Q8_0, N, K, seed=9)
    x = synth.activations(1, K, seed=10)
    a1 = orc.quantize_q8_1(x)
    a2 = orc.quantize_q8_1(2 * x)     # scaling by 2 is exact in Q8_1 (codes equal, d doubles)
    y1 = orc.gemv_exact(Q8_0, w, a1, 1, N, K)
    y2 = orc.gemv_exact(Q8_0, w, a2, 1, N, K)
    assert np.allclose(y2, 2 * y1, rtol=1e-12)
    az = orc.quantize_q8_1(np.zeros((1, K), np.float32))
    assert not orc.gemv_exact(Q8_0, w, az, 1, N, K).any()
    w0 = w.copy()
    w0.reshape(-1, 34)[:, 0:2] = 0   # d = 0 -> y = 0
    assert not orc.gemv_exact(Q8_0, w0, a1, 1, N, K).any()


@pytest.mark.parametrize("qtype", [Q4_K, Q6_K])
def test_gemv_reference_patterns(orc, qtype):
    """The reference's deterministic weight patterns (FillQuantizedRows,
    MakeQ4Rows) with its sin-wave activations; its own margin is 8e-2
    absolute (test_native_forward.cpp:4620-4739)."""
    K, N, M = 512, 8, 2
    w = qref.fill_quantized_rows(qtype, N, K // 256)
    x = np.stack([qref.make_wave_tensor(K, 0.5, 0.0), qref.make_wave_tensor(K, 0.25, 0.1)])
    a = orc.quantize_q8_1(x)
    y = orc.gemv_q8_1(qtype, w, a, M, N, K)
    ye = orc.gemv_exact(qtype, w, a, M, N, K)
    assert np.abs(y - ye).max() <= 8e-2
    assert np.all(np.abs(y - ye).max(axis=1) <= orc.row_norm_tolerance(ye, 1e-4))
    if qtype == Q4_K:
        w2 = qref.make_q4_rows(N, K // 256, seed=3)
        y2 = orc.gemv_q8_1(Q4_K, w2, a, M, N, K)
        assert np.abs(y2 - orc.gemv_exact(Q4_K, w2, a, M, N, K)).max() <= 8e-2


@pytest.mark.parametrize("qtype", [Q4_K, Q6_K, Q8_0])
def test_ggml_semantics_baseline(orc, qtype):
    """The CPU baseline (ggml's Q8_K / Q8_0 activation formats) against the
    unquantized fp64 product.  ggml itself is absent: parity unpinned beyond
    this tolerance."""
    from inferflux_amd import synth
    K, N, M = 1024, 32, 2
    w = synth.blocks(qtype, N, K, seed=12)
    x = synth.activations(M, K, seed=13)
    y = orc.ggml_cpu_gemv(qtype, w, x, N)
    want = x.astype(np.float64) @ qref.dequant_f64(qtype, w, N, K).T
    assert np.all(np.abs(y - want).max(axis=1) <= orc.row_norm_tolerance(want, 1e-2))


def test_golden_gemv_fixture(orc):
    """Committed small-case vectors (tests/golden/make_golden.py)."""
    z = np.load(os.path.join(GOLDEN, "gemv_small.npz"))
    for qtype in (Q4_K, Q6_K, Q8_0):
        w, x = z[f"w_{qtype}"], z[f"x_{qtype}"]
        M, K = x.shape
        N = w.shape[0]
        a = orc.quantize_q8_1(x)
        assert np.array_equal(a, z[f"a_{qtype}"])
        assert np.array_equal(orc.dequantize(qtype, w, N, K), z[f"wf_{qtype}"])
        y = orc.gemv_exact(qtype, w, a, M, N, K)
        assert np.allclose(y, z[f"y_{qtype}"], rtol=1e-12, atol=0)


def test_q8_1_double_rounding_fixture(orc):
    """s is rounded to fp32 first, then to fp16 (fused_dequant_gemv.cuh:650)."""
    z = np.load(os.path.join(GOLDEN, "gemv_small.npz"))
    assert np.array_equal(orc.quantize_q8_1(z["dr_x"]), z["dr_q8_1"])


# ------------------------------------------------ fused Q8_1 producers
def test_rmsnorm_values_vs_fp64(orc):
    rng = np.random.default_rng(5)
    x = (rng.standard_normal((3, 2048)) * 3).astype(np.float32)
    w = (rng.standard_normal(2048) * 0.5).astype(np.float16)
    y = orc.rmsnorm_values(x, w, 1e-5)
    xd = x.astype(np.float64)
    ref = xd / np.sqrt((xd * xd).mean(axis=1, keepdims=True) + 1e-5) * w.astype(np.float64)
    assert np.allclose(y, ref, rtol=4e-7, atol=1e-30)
    # fp16 residual input is widened exactly
    x16 = x.astype(np.float16)
    assert np.array_equal(orc.rmsnorm_values(x16, w, 1e-5),
                          orc.rmsnorm_values(x16.astype(np.float32), w, 1e-5))


def test_rmsnorm_quantize_is_quantizer_of_values(orc):
    rng = np.random.default_rng(6)
    x = rng.standard_normal((2, 1024)).astype(np.float32)
    w = rng.uniform(0.5, 1.5, 1024).astype(np.float16)
    assert np.array_equal(orc.rmsnorm_quantize_q8_1(x, w, 1e-6),
                          orc.quantize_q8_1(orc.rmsnorm_values(x, w, 1e-6)))


def test_rmsnorm_exact_kat(orc):
    """x = +-1 and eps = 0: sum(x^2) = K, rms = 1 exactly, y = x * w."""
    rng = np.random.default_rng(7)
    x = np.where(rng.random((2, 512)) < 0.5, -1.0, 1.0).astype(np.float32)
    w = rng.standard_normal(512).astype(np.float16)
    y = orc.rmsnorm_values(x, w, 0.0)
    assert np.array_equal(y, x * w.astype(np.float32))


def test_silu_mul_values_vs_fp64(orc):
    rng = np.random.default_rng(8)
    g = (rng.standard_normal(4096) * 3).astype(np.float32)
    u = rng.standard_normal(4096).astype(np.float32)
    y = orc.silu_mul_values(g, u)
    gd = g.astype(np.float64)
    ref = gd / (1 + np.exp(-gd)) * u
    assert np.allclose(y, ref, rtol=3e-7, atol=1e-30)
    # silu(0) = 0; silu(g) = g in fp32 once exp(-g) < 2^-24
    z = orc.silu_mul_values(np.array([0.0, 20.0, 30.0], np.float32), np.array([5.0, 3.0, -2.0], np.float32))
    assert np.array_equal(z, np.array([0.0, 60.0, -60.0], np.float32))


# ------------------------------------------- packed (row-symmetric) activations
def test_quantize_rows_symmetric_reference_kat(orc):
    """The reference's contract test (tests/unit/test_native_forward.cpp:
    7181-7238): two rows of four, scales 4/127 and 3/127, -2 and 1.5 land on
    the tie 63.5 and round to even."""
    x = np.array([[-4.0, -2.0, 0.0, 4.0], [0.0, 1.5, -1.5, 3.0]], np.float32)
    codes, scales = orc.quantize_rows_symmetric(x)
    assert codes.tolist() == [[-127, -64, 0, 127], [0, 64, -64, 127]]
    assert scales[0] == np.float32(4.0) / np.float32(127.0)
    assert scales[1] == np.float32(3.0) / np.float32(127.0)


def test_quantize_rows_symmetric_ties_zero_and_clamp(orc):
    # amax 127 -> scale 1 exactly: codes are rint(x), ties to even
    x = np.array([[127.0, 63.5, 62.5, -0.5, 0.49, -126.5, 1.5, 2.5]], np.float32)
    codes, scales = orc.quantize_rows_symmetric(x)
    assert scales[0] == 1.0
    assert codes.tolist() == [[127, 64, 62, 0, 0, -126, 2, 2]]
    codes, scales = orc.quantize_rows_symmetric(np.zeros((2, 64), np.float32))
    assert scales.tolist() == [0.0, 0.0] and not codes.any()


def test_quantize_rows_symmetric_properties(orc):
    rng = np.random.default_rng(7)
    x = (rng.standard_normal((16, 1000)) * rng.uniform(1e-3, 1e3, (16, 1))).astype(np.float32)
    codes, scales = orc.quantize_rows_symmetric(x)
    amax = np.abs(x).max(axis=1)
    assert np.array_equal(scales, (amax / np.float32(127)).astype(np.float32))
    # the largest magnitude maps to +-127; every code is within half a step
    idx = np.abs(x).argmax(axis=1)
    assert np.array_equal(np.abs(codes[np.arange(16), idx]), np.full(16, 127))
    err = np.abs(x.astype(np.float64) - codes * scales[:, None].astype(np.float64))
    assert np.all(err <= 0.5 * scales[:, None] * (1 + 1e-6))
    # sign symmetry
    c2, s2 = orc.quantize_rows_symmetric(-x)
    assert np.array_equal(c2, -codes) and np.array_equal(s2, scales)


def test_silu_mul_quantize_rows_symmetric_reference_kat(orc):
    """The reference's SwiGLU quantization test (test_native_forward.cpp:
    7634-7700): codes lrint(y / scale) with scale = max|y| / 127."""
    g = np.array([[-1.0, 0.0, 1.0, 2.0, -2.0, 0.5, -0.5, 3.0]], np.float32)
    u = np.array([[1.0, 1.0, 1.0, 1.0, 0.5, 2.0, 4.0, 1.0]], np.float32)
    codes, scales = orc.silu_mul_quantize_rows_symmetric(g, u)
    assert codes.tolist() == [[-12, 0, 32, 78, -5, 28, -34, 127]]
    y = g.astype(np.float64) / (1 + np.exp(-g.astype(np.float64))) * u
    assert abs(scales[0] - np.abs(y).max() / 127) <= 1e-7


@pytest.mark.parametrize("qtype,K", [(Q4_K, 512), (Q6_K, 768), (Q8_0, 160), (Q8_K, 512)])
def test_gemv_packed_equals_q8_1_gemv(orc, qtype, K):
    """With a power-of-two row scale both activation formats hold the same
    values exactly (Q8_1 blocks with d = scale and the same codes), so the
    packed GEMV equals the pinned Q8_1 GEMV up to fp64 summation order."""
    from inferflux_amd import synth
    M, N = 3, 40
    rng = np.random.default_rng(K)
    codes = rng.integers(-127, 128, (M, K)).astype(np.int8)
    scales = np.array([2.0**-4, 2.0**-7, 1.0], np.float32)
    a = np.zeros((M, K // 32, 36), np.uint8)
    a[:, :, 0:2] = np.frombuffer(np.repeat(scales.astype(np.float16), K // 32).tobytes(),
                                 np.uint8).reshape(M, K // 32, 2)
    a[:, :, 4:36] = codes.reshape(M, K // 32, 32).view(np.uint8)
    w = synth.blocks(qtype, N, K, seed=K + 1)
    y_packed = orc.gemv_packed_exact(qtype, w, codes, scales, M, N, K)
    y_q8_1 = orc.gemv_exact(qtype, w, a.reshape(M, -1), M, N, K)
    assert np.allclose(y_packed, y_q8_1, rtol=1e-12, atol=1e-12 * np.abs(y_q8_1).max())


def test_gemv_packed_closed_form(orc):
    """Q8_0 rows of code 1 with d = 1: y = scale * sum(codes)."""
    M, N, K = 2, 3, 64
    w = np.zeros((N * K // 32, 34), np.uint8)
    w[:, 0:2] = np.frombuffer(np.float16(1.0).tobytes(), np.uint8)
    w[:, 2:34] = 1
    rng = np.random.default_rng(3)
    codes = rng.integers(-127, 128, (M, K)).astype(np.int8)
    scales = np.array([0.5, 3.0], np.float32)
    y = orc.gemv_packed_exact(Q8_0, w, codes, scales, M, N, K)
    want = scales[:, None] * codes.sum(axis=1, dtype=np.int64)[:, None]
    assert np.array_equal(y, np.repeat(want, N, axis=1).astype(np.float64))
