"""GPU parity: the HIP kernels (through the C ABI) against the CPU oracle on
identical seeded inputs.

Bars: Q8_1 codes/scales and dequantized values bit-exact; GEMV/GEMM fp32
outputs within 1e-3 * ||y_row||_2 (per output row m, over its N values) of
the fp64 oracle, as the contract states.  Full benchmark sizes are checked
on sampled weight rows (the product restricted to a row subset is the
product of the row subset), so the oracle finishes in seconds.
"""
import numpy as np
import pytest

from tests import qref

pytestmark = pytest.mark.gpu

Q8_0, Q4_K, Q5_K, Q6_K, Q8_K = 8, 12, 13, 14, 15
TOL = 1e-3


@pytest.fixture(scope="module")
def dev():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda:0")


def up(arr, dev):
    import torch
    return torch.from_numpy(np.ascontiguousarray(arr)).to(dev)


def down(t):
    import torch
    torch.cuda.synchronize()
    return t.cpu().numpy()


def note(msg):
    print(msg, flush=True)


def check_h_propagated(h, g, u, tol=1e-3):
    """h = silu(g) * u from two GEMV outputs, each held to the contract's
    tol * ||row||_2: the bar on h is that error carried through the product,
    |dh| <= |silu'(g) u| tol ||g_row|| + |silu(g)| tol ||u_row||.  (A row of h
    dominated by one element can exceed tol * ||h_row|| with g and u inside
    their own bars: the fp16-dequant GEMV rounds each weight to fp16.)"""
    with np.errstate(over="ignore"):
        sg = 1.0 / (1.0 + np.exp(-g))
    dsilu = sg * (1.0 + g * (1.0 - sg))
    eg = tol * np.linalg.norm(g, axis=1, keepdims=True)
    eu = tol * np.linalg.norm(u, axis=1, keepdims=True)
    bound = np.abs(dsilu * u) * eg + np.abs(g * sg) * eu + eg * eu
    err = np.abs(np.asarray(h, np.float64) - g * sg * u)
    assert np.all(err <= bound), f"max err / bound {(err / bound).max()}"


def same_slot_waves(grouped, fused):
    """True when a grouped launch and the fused gate/up/SiLU launch are both
    slot-packed MFMA GEMVs with the same waves per projection (the third
    template argument), i.e. they add the same partial sums in one order."""
    def waves(name):
        if not name.startswith("k_gemv_slot<"):
            return None
        return name[len("k_gemv_slot<"):-1].split(",")[2]
    return waves(grouped) is not None and waves(grouped) == waves(fused)


def check_rows(y, ye, tol=TOL):
    y = np.asarray(y, np.float64)
    err = np.abs(y - ye).max(axis=1)
    lim = tol * np.linalg.norm(ye, axis=1)
    assert np.all(err <= lim), f"max err {err.max()} vs limit {lim.min()}"
    return (err / np.maximum(lim / tol, 1e-30)).max()


# -------------------------------------------------------------- quantizer
@pytest.mark.parametrize("M,K,outl", [(1, 32, 0.0), (1, 2048, 0.0), (4, 2048, 0.01),
                                      (8, 11008, 0.0), (3, 13824, 0.01), (512, 5120, 0.01)])
def test_quantize_q8_1_bit_exact(orc, dev, M, K, outl):
    from inferflux_amd import ops, synth
    note(f"quantize M={M} K={K}")
    x = synth.activations(M, K, seed=M * 7 + K, outlier_frac=outl)
    x[0, :32] = 0.0  # an all-zero block
    got = down(ops.quantize_q8_1(up(x, dev)))
    want = orc.quantize_q8_1(x)
    bad = np.nonzero((got != want).reshape(-1, 36).any(axis=1))[0]
    assert bad.size == 0, f"{bad.size} blocks differ, first {bad[0]}: {got.reshape(-1, 36)[bad[0]]} vs {want.reshape(-1, 36)[bad[0]]}"


def test_quantize_double_rounding_regression(dev):
    """Blocks where fusing d*sum into the fp16 conversion changes s."""
    import os
    from inferflux_amd import ops
    z = np.load(os.path.join(os.path.dirname(__file__), "golden", "gemv_small.npz"))
    assert np.array_equal(down(ops.quantize_q8_1(up(z["dr_x"], dev))), z["dr_q8_1"])


def test_quantize_q8_1_f16_input(orc, dev):
    from inferflux_amd import ops
    x = (np.random.default_rng(4).standard_normal((5, 1024)) * 4).astype(np.float16)
    got = down(ops.quantize_q8_1(up(x, dev)))
    assert np.array_equal(got, orc.quantize_q8_1(x))


def test_quantize_reference_kat(dev):
    import json
    import os
    from inferflux_amd import ops
    kat = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "q8_1_kat.json")))
    for case in kat["cases"]:
        x = np.array(case["x"], np.float32).reshape(1, -1)
        a = down(ops.quantize_q8_1(up(x, dev)))
        d, s, q = qref.q8_1_fields(a, 1, x.shape[1])
        assert q.ravel().tolist() == case["q"] == case["q_ref_test_formula"]
        assert d.view(np.uint16).ravel().tolist() == case["d_bits"]
        assert s.view(np.uint16).ravel().tolist() == case["s_bits"]


# ---------------------------------------------------------------- dequant
@pytest.mark.parametrize("qtype,n,K", [(Q4_K, 33, 2048), (Q6_K, 17, 11008), (Q8_0, 9, 2080),
                                      (Q5_K, 9, 2048), (Q8_K, 7, 1024), (Q8_0, 3, 96)])
def test_dequant_bit_exact(orc, dev, qtype, n, K):
    import torch
    from inferflux_amd import ops, synth
    note(f"dequant type={qtype} n={n} K={K}")
    w = synth.blocks(qtype, n, K, seed=qtype)
    want = orc.dequantize(qtype, w, n, K)
    got = down(ops.dequantize(qtype, up(w, dev), n, K))
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    got16 = down(ops.dequantize(qtype, up(w, dev), n, K, out_dtype=torch.float16))
    assert np.array_equal(got16.view(np.uint16), orc.f32_to_f16_bits(want))


# ---------------------------------------------------------------- GEMV
CASES = []
for qt in (Q4_K, Q6_K, Q8_0):
    for M in (1, 2, 3, 4, 5, 8):
        CASES.append((qt, M, 1000, 2048))
    CASES.append((qt, 1, 37, 5120))
    CASES.append((qt, 8, 129, 11008 if qt != Q6_K else 13824))
CASES.append((Q8_0, 3, 50, 96))     # K not a multiple of 256
CASES.append((Q4_K, 3, 300, 5120))  # activations-in-LDS GEMV, full-wave rows
CASES.append((Q4_K, 4, 16400, 2048))  # activations-in-LDS GEMV, M = 4 wide launch
CASES.append((Q4_K, 2, 8200, 5120))  # quarter-wave rows, two columns
CASES.append((Q4_K, 1, 100, 3072))   # quarter-wave rows, 3 slices per lane
CASES += [(Q6_K, 1, 301, 11008), (Q4_K, 1, 77, 11008)]  # wide slices, 3 waves per row group
# slot-packed MFMA GEMV (5 <= M <= 16): 8- and 16-row slots, ragged N, one
# super-block per row, a single row
CASES += [(Q4_K, 6, 33, 256), (Q6_K, 7, 64, 512), (Q4_K, 12, 1000, 2048),
          (Q6_K, 16, 1000, 2048), (Q4_K, 16, 31, 5120), (Q6_K, 9, 1, 1024),
          (Q6_K, 13, 77, 11008)]
for qt in (Q5_K, Q8_K):             # GEMV-only types, M <= 64
    for M in (1, 2, 3, 8, 17, 64):
        CASES.append((qt, M, 300, 2048))
    CASES.append((qt, 1, 37, 5120))


@pytest.mark.parametrize("qtype,M,N,K", CASES)
def test_gemv_parity(orc, dev, qtype, M, N, K):
    from inferflux_amd import ops, synth
    note(f"gemv type={qtype} M={M} N={N} K={K}")
    w = synth.blocks(qtype, N, K, seed=N + K)
    x = synth.activations(M, K, seed=M + K, outlier_frac=0.01)
    a = orc.quantize_q8_1(x)
    y = down(ops.qgemv(qtype, up(w, dev), up(a, dev), M, N, K))
    check_rows(y, orc.gemv_exact(qtype, w, a, M, N, K))


@pytest.mark.parametrize("qtype", [Q4_K, Q6_K])
def test_gemv_reference_patterns(orc, dev, qtype):
    """The reference tests' deterministic rows and sin-wave activations
    (test_native_forward.cpp:47,112-160) with its 8e-2 absolute margin."""
    from inferflux_amd import ops
    K, N, M = 512, 64, 2
    w = qref.fill_quantized_rows(qtype, N, K // 256)
    x = np.stack([qref.make_wave_tensor(K, 0.5), qref.make_wave_tensor(K, 0.25, 0.1)])
    a = orc.quantize_q8_1(x)
    y = down(ops.qgemv(qtype, up(w, dev), up(a, dev), M, N, K))
    ye = orc.gemv_exact(qtype, w, a, M, N, K)
    assert np.abs(y - ye).max() <= 8e-2
    check_rows(y, ye)


@pytest.mark.parametrize("qtype", [Q4_K, Q6_K, Q8_0, Q5_K, Q8_K])
@pytest.mark.parametrize("M", [1, 3, 8, 24])
def test_epilogues(orc, dev, qtype, M):
    """Accumulate (GemvQ8_1Accum / AccumF32) and bias (GemvQ8_1WithBias),
    fp32 and fp16 outputs."""
    import torch
    from inferflux_amd import ops, synth
    note(f"epilogue type={qtype} M={M}")
    N, K = 300, 1024
    w = synth.blocks(qtype, N, K, seed=3)
    a = orc.quantize_q8_1(synth.activations(M, K, seed=4))
    ye = orc.gemv_exact(qtype, w, a, M, N, K)
    base = np.random.default_rng(5).standard_normal((M, N)).astype(np.float32)
    bias = np.random.default_rng(6).standard_normal(N).astype(np.float32)
    W, A = up(w, dev), up(a, dev)
    y = ops.qgemv(qtype, W, A, M, N, K, out=up(base, dev), mode=ops.ACCUM)
    check_rows(down(y), ye + base)
    y = ops.qgemv(qtype, W, A, M, N, K, mode=ops.BIAS, bias=up(bias, dev))
    check_rows(down(y), ye + bias[None, :])
    y16 = ops.qgemv(qtype, W, A, M, N, K, out_dtype=torch.float16)
    check_rows(down(y16).astype(np.float64), ye, tol=2e-3)
    b16 = base.astype(np.float16)
    y16 = ops.qgemv(qtype, W, A, M, N, K, out=up(b16, dev), mode=ops.ACCUM)
    check_rows(down(y16).astype(np.float64), ye + b16.astype(np.float64), tol=2e-3)


@pytest.mark.parametrize("qtype,M,N,K", [
    (Q4_K, 6, 8200, 512),    # slot-packed GEMV, wide launch (ragged last row group)
    (Q6_K, 8, 8195, 256),    # one super-block per row
    (Q6_K, 5, 96, 8192),     # long K, few rows: split over workgroups (atomics)
    (Q4_K, 8, 33, 11008),
    (Q6_K, 3, 200, 11008),   # long K at M = 3 / 4 (the down projection)
    (Q6_K, 4, 64, 8192),
])
def test_slot_epilogues(orc, dev, qtype, M, N, K):
    """Store, accumulate and bias modes of the slot-packed MFMA GEMV, with
    and without the workgroup split of K; fp16 outputs (never split), stored
    and accumulated."""
    import torch
    from inferflux_amd import ops, synth
    note(f"slot epilogue type={qtype} M={M} N={N} K={K}")
    w = synth.blocks(qtype, N, K, seed=N + 7)
    a = orc.quantize_q8_1(synth.activations(M, K, seed=K + 1, outlier_frac=0.01))
    ye = orc.gemv_exact(qtype, w, a, M, N, K)
    base = np.random.default_rng(5).standard_normal((M, N)).astype(np.float32)
    bias = np.random.default_rng(6).standard_normal(N).astype(np.float32)
    W, A = up(w, dev), up(a, dev)
    # a store after garbage in the output: the split path zeroes it first
    y = ops.qgemv(qtype, W, A, M, N, K, out=torch.full((M, N), 7.0, device=dev))
    check_rows(down(y), ye)
    y = ops.qgemv(qtype, W, A, M, N, K, out=up(base, dev), mode=ops.ACCUM)
    check_rows(down(y), ye + base)
    y = ops.qgemv(qtype, W, A, M, N, K, mode=ops.BIAS, bias=up(bias, dev))
    check_rows(down(y), ye + bias[None, :])
    y16 = ops.qgemv(qtype, W, A, M, N, K, out_dtype=torch.float16)
    check_rows(down(y16).astype(np.float64), ye, tol=2e-3)
    # fp16 accumulate: unsplit, the added term loaded ahead of the weights
    b16 = base.astype(np.float16)
    y16 = ops.qgemv(qtype, W, A, M, N, K, out=up(b16, dev), mode=ops.ACCUM)
    check_rows(down(y16).astype(np.float64), ye + b16.astype(np.float64), tol=2e-3)


# ------------------------------------------------------------ MFMA GEMM
@pytest.mark.parametrize("qtype,M,N,K", [
    (Q4_K, 9, 200, 512), (Q4_K, 16, 256, 2048), (Q4_K, 32, 130, 1024), (Q4_K, 130, 300, 768),
    (Q6_K, 16, 256, 2048), (Q6_K, 33, 100, 1024), (Q6_K, 200, 129, 512),
    (Q8_0, 16, 256, 2048), (Q8_0, 64, 77, 512), (Q8_0, 10, 40, 160),
])
def test_gemm_parity(orc, dev, qtype, M, N, K):
    from inferflux_amd import ops, synth
    note(f"gemm type={qtype} M={M} N={N} K={K}")
    w = synth.blocks(qtype, N, K, seed=N * 3 + K)
    a = orc.quantize_q8_1(synth.activations(M, K, seed=M, outlier_frac=0.01))
    ye = orc.gemv_exact(qtype, w, a, M, N, K)
    W, A = up(w, dev), up(a, dev)
    check_rows(down(ops.qgemv(qtype, W, A, M, N, K)), ye)
    check_rows(down(ops.qgemv(qtype, W, A, M, N, K, prefill=True)), ye)


@pytest.mark.parametrize("qtype,M,N,K", [
    (Q4_K, 130, 300, 768), (Q6_K, 200, 129, 512), (Q8_0, 64, 77, 512),
])
def test_gemm_int8_kernel_parity(orc, dev, qtype, M, N, K):
    """The integer-exact int8 MFMA GEMM, which the dispatch no longer picks
    from 128 rows on, stays reachable and correct."""
    from inferflux_amd import ops, synth
    note(f"gemm int8 type={qtype} M={M} N={N} K={K}")
    w = synth.blocks(qtype, N, K, seed=N * 3 + K)
    a = orc.quantize_q8_1(synth.activations(M, K, seed=M, outlier_frac=0.01))
    ye = orc.gemv_exact(qtype, w, a, M, N, K)
    y = ops.qgemm_prefill_kernel(qtype, up(w, dev), up(a, dev), M, N, K, ops.PREFILL_INT8)
    check_rows(down(y), ye)


# fp16 GEMM with in-kernel dequant: ragged M/N edges, one-stage K, forced
# K splits (fp32 atomics), every output mode and fp16 output.
@pytest.mark.parametrize("qtype,M,N,K,splits", [
    (Q4_K, 1, 64, 256, 0), (Q4_K, 256, 256, 256, 0), (Q4_K, 300, 513, 1024, 0),
    (Q4_K, 77, 100, 2048, 3), (Q6_K, 129, 257, 512, 0), (Q6_K, 512, 64, 2048, 5),
    (Q8_0, 200, 300, 192, 0), (Q8_0, 33, 64, 512, 2), (Q6_K, 40, 300, 256, 4),
])
def test_gemm_f16_parity(orc, dev, qtype, M, N, K, splits):
    import torch
    from inferflux_amd import ops, synth
    note(f"gemm f16 type={qtype} M={M} N={N} K={K} splits={splits}")
    w = synth.blocks(qtype, N, K, seed=N * 7 + K)
    a = orc.quantize_q8_1(synth.activations(M, K, seed=M + 1, outlier_frac=0.01))
    ye = orc.gemv_exact(qtype, w, a, M, N, K)
    W, A = up(w, dev), up(a, dev)
    rng = np.random.default_rng(M)
    base = rng.standard_normal((M, N)).astype(np.float32)
    bias = rng.standard_normal(N).astype(np.float32)
    f = ops.PREFILL_F16
    y = ops.qgemm_prefill_kernel(qtype, W, A, M, N, K, f, splits,
                                 out=torch.full((M, N), 7.0, device=dev))
    check_rows(down(y), ye)
    y = ops.qgemm_prefill_kernel(qtype, W, A, M, N, K, f, splits, out=up(base, dev),
                                 mode=ops.ACCUM)
    check_rows(down(y), ye + base)
    y = ops.qgemm_prefill_kernel(qtype, W, A, M, N, K, f, splits, mode=ops.BIAS,
                                 bias=up(bias, dev))
    check_rows(down(y), ye + bias[None, :])
    y16 = ops.qgemm_prefill_kernel(qtype, W, A, M, N, K, f, splits, out_dtype=torch.float16)
    check_rows(down(y16).astype(np.float64), ye, tol=2e-3)
    b16 = up(bias.astype(np.float16), dev)
    y16 = ops.qgemm_prefill_kernel(qtype, W, A, M, N, K, f, splits, out_dtype=torch.float16,
                                   mode=ops.BIAS, bias=b16)
    check_rows(down(y16).astype(np.float64), ye + bias.astype(np.float16)[None, :], tol=2e-3)


# decode-batch fp16 dequant kernel: every M up to 32, forced K splits
# (fp32 atomics after a zero fill), all output modes and fp16 output.
@pytest.mark.parametrize("qtype,M,N,K,splits", [
    (Q4_K, 1, 64, 256, 0), (Q4_K, 3, 300, 1024, 0), (Q4_K, 8, 1000, 2048, 0),
    (Q4_K, 16, 129, 512, 2), (Q4_K, 32, 256, 1536, 3), (Q4_K, 13, 77, 768, 1),
    (Q6_K, 5, 130, 512, 0), (Q6_K, 16, 256, 2048, 4), (Q6_K, 32, 65, 256, 0),
    (Q8_0, 4, 200, 512, 0), (Q8_0, 24, 129, 1024, 2), (Q8_0, 32, 64, 256, 1),
])
def test_gemv_dq_parity(orc, dev, qtype, M, N, K, splits):
    import torch
    from inferflux_amd import ops, synth
    note(f"gemv dq type={qtype} M={M} N={N} K={K} splits={splits}")
    w = synth.blocks(qtype, N, K, seed=N * 5 + K + M)
    a = orc.quantize_q8_1(synth.activations(M, K, seed=M + 7, outlier_frac=0.01))
    ye = orc.gemv_exact(qtype, w, a, M, N, K)
    W, A = up(w, dev), up(a, dev)
    rng = np.random.default_rng(M + N)
    base = rng.standard_normal((M, N)).astype(np.float32)
    bias = rng.standard_normal(N).astype(np.float32)
    kern = ops.DECODE_DQ_F16
    y = ops.qgemm_prefill_kernel(qtype, W, A, M, N, K, kern, splits,
                                 out=torch.full((M, N), 7.0, device=dev))
    check_rows(down(y), ye)
    y = ops.qgemm_prefill_kernel(qtype, W, A, M, N, K, kern, splits, out=up(base, dev),
                                 mode=ops.ACCUM)
    check_rows(down(y), ye + base)
    y = ops.qgemm_prefill_kernel(qtype, W, A, M, N, K, kern, splits, mode=ops.BIAS,
                                 bias=up(bias, dev))
    check_rows(down(y), ye + bias[None, :])
    if (K // 256) * 256 * (M + 1) * 2 <= 65536 - 16 * (M + 1):  # one activation stage
        y16 = ops.qgemm_prefill_kernel(qtype, W, A, M, N, K, kern, splits,
                                       out_dtype=torch.float16)
        check_rows(down(y16).astype(np.float64), ye, tol=2e-3)
    else:  # fp16 outputs cannot be split over K
        with pytest.raises(ops.NotHandled):
            ops.qgemm_prefill_kernel(qtype, W, A, M, N, K, kern, splits, out_dtype=torch.float16)


@pytest.mark.parametrize("qtype,M,N,K", [(Q4_K, 128, 16400, 512), (Q4_K, 256, 16384, 256),
                                         (Q6_K, 129, 16384, 256), (Q8_0, 200, 16500, 192),
                                         (Q6_K, 512, 320, 4096)])
def test_gemm_f16_workspace(orc, dev, qtype, M, N, K):
    """The activations converted once into a caller workspace give the same
    bits as the per-tile conversion (fp16 output: no split-K atomics), and
    fp32 outputs pass the oracle bar; a short or misaligned workspace is
    refused.  Below N = 16384 no workspace is used and the call is the plain
    prefill GEMM."""
    import torch
    from inferflux_amd import ops, synth
    note(f"gemm_f16 workspace type={qtype} M={M} N={N} K={K}")
    w = synth.blocks(qtype, N, K, seed=M + N)
    a = orc.quantize_q8_1(synth.activations(M, K, seed=K + 1, outlier_frac=0.01))
    need = ops.prefill_workspace_bytes(qtype, M, N, K)
    assert need == (M * K * 2 if N >= 16384 else 0)
    ws = torch.empty(max(need, 16) // 2 + 8, dtype=torch.float16, device=dev)
    W, A = up(w, dev), up(a, dev)
    y16 = ops.qgemv(qtype, W, A, M, N, K, out_dtype=torch.float16, prefill=True)
    y16w = ops.qgemm_prefill_ws(qtype, W, A, M, N, K, ws, out_dtype=torch.float16)
    assert np.array_equal(down(y16w).view(np.uint16), down(y16).view(np.uint16))
    y = ops.qgemm_prefill_ws(qtype, W, A, M, N, K, ws)
    check_rows(down(y), orc.gemv_exact(qtype, w, a, M, N, K))
    if need:
        with pytest.raises(ops.NotHandled):
            ops.qgemm_prefill_ws(qtype, W, A, M, N, K, ws[: need // 2 - 1])
        with pytest.raises(ops.NotHandled):
            ops.qgemm_prefill_ws(qtype, W, A, M, N, K, ws[1:])
    # below the prefill range there is no workspace
    assert ops.prefill_workspace_bytes(qtype, 32, N, K) == 0


def test_gemm_f16_rejects_ragged_k(dev):
    import torch
    from inferflux_amd import ops
    W = torch.zeros(4096, dtype=torch.uint8, device=dev)
    A = torch.zeros(4096, dtype=torch.uint8, device=dev)
    # Q8_0 with K % 64 != 0 has no fp16 stage layout: not handled
    with pytest.raises(ops.NotHandled) as e:
        ops.qgemm_prefill_kernel(Q8_0, W, A, 2, 4, 96, ops.PREFILL_F16)
    assert e.value.status == 2


def test_prefill_small_m_via_prefill_entry(orc, dev):
    from inferflux_amd import ops, synth
    qtype, M, N, K = Q4_K, 3, 64, 512
    w = synth.blocks(qtype, N, K, seed=1)
    a = orc.quantize_q8_1(synth.activations(M, K, seed=2))
    y = down(ops.qgemv(qtype, up(w, dev), up(a, dev), M, N, K, prefill=True))
    check_rows(y, orc.gemv_exact(qtype, w, a, M, N, K))


# ------------------------------------------- benchmark sizes, sampled rows
def _sampled(orc, dev, qtype, M, N, K, seed, outl=0.0, rows=256):
    from inferflux_amd import ops, synth
    note(f"full-size type={qtype} M={M} N={N} K={K}")
    w = synth.blocks(qtype, N, K, seed=seed)
    x = synth.activations(M, K, seed=seed + 1, outlier_frac=outl)
    A = ops.quantize_q8_1(up(x, dev))
    a = down(A)
    assert np.array_equal(a, orc.quantize_q8_1(x))
    y = down(ops.qgemv(qtype, up(w, dev), A, M, N, K))
    idx = np.unique(np.concatenate([[0, N - 1], np.random.default_rng(seed).choice(N, rows)]))
    ye = orc.gemv_exact(qtype, w[idx], a, M, len(idx), K)
    # the tolerance is relative to the norm of the whole output row; the
    # sampled norm scales it down by sqrt(len(idx)/N), which is stricter
    check_rows(y[:, idx], ye)
    assert np.isfinite(y).all()


@pytest.mark.parametrize("qtype", [Q4_K, Q6_K, Q8_0])
def test_gemm_large_tiles(orc, dev, qtype):
    """The int8 MFMA GEMM on a grid of >= 512 tiles of 128 x 128 (M = 1000,
    N = 8190: 8 x 64 tiles), which takes its large-tile instance
    k_gemm_mfma<QT, 2> (the small parity cases above run 64 x 64 tiles);
    ragged M and N edges; store, accumulate, bias and fp16 outputs."""
    import torch
    from inferflux_amd import ops, synth
    M, N, K = 1000, 8190, 512
    note(f"gemm int8 large tiles type={qtype} M={M} N={N} K={K}")
    w = synth.blocks(qtype, N, K, seed=21)
    a = orc.quantize_q8_1(synth.activations(M, K, seed=22, outlier_frac=0.01))
    W, A = up(w, dev), up(a, dev)
    idx = np.unique(np.concatenate([[0, N - 1], np.random.default_rng(21).choice(N, 128)]))
    ye = orc.gemv_exact(qtype, w[idx], a, M, len(idx), K)
    rng = np.random.default_rng(23)
    base = rng.standard_normal((M, N)).astype(np.float32)
    bias = rng.standard_normal(N).astype(np.float32)
    kern = ops.PREFILL_INT8
    with ops.launch_log() as lg:
        y = ops.qgemm_prefill_kernel(qtype, W, A, M, N, K, kern,
                                     out=torch.full((M, N), 7.0, device=dev))
    assert lg.kernels == [f"k_gemm_mfma<{qtype},2,0>"]
    check_rows(down(y)[:, idx], ye)
    y = ops.qgemm_prefill_kernel(qtype, W, A, M, N, K, kern, out=up(base, dev), mode=ops.ACCUM)
    check_rows(down(y)[:, idx], ye + base[:, idx])
    y = ops.qgemm_prefill_kernel(qtype, W, A, M, N, K, kern, mode=ops.BIAS, bias=up(bias, dev))
    check_rows(down(y)[:, idx], ye + bias[None, idx])
    with ops.launch_log() as lg:
        y16 = ops.qgemm_prefill_kernel(qtype, W, A, M, N, K, kern, out_dtype=torch.float16)
    assert lg.kernels == [f"k_gemm_mfma<{qtype},2,1>"]
    check_rows(down(y16)[:, idx].astype(np.float64), ye, tol=2e-3)


@pytest.mark.parametrize("M", [1, 8])
def test_config1_q4k_gemv(orc, dev, M):
    _sampled(orc, dev, Q4_K, M, 11008, 2048, seed=0, rows=11008)


@pytest.mark.parametrize("M", [1, 8])
@pytest.mark.parametrize("qtype", [Q8_0, Q6_K])
def test_config3_lm_head(orc, dev, qtype, M):
    _sampled(orc, dev, qtype, M, 151936, 2048, seed=3)


@pytest.mark.parametrize("M", [16, 32])
def test_config4_14b_down_and_gate(orc, dev, M):
    _sampled(orc, dev, Q6_K, M, 5120, 13824, seed=4)
    _sampled(orc, dev, Q4_K, M, 13824, 5120, seed=4)


@pytest.mark.parametrize("qtype,N,K", [(Q4_K, 27648, 5120), (Q6_K, 5120, 27648)])
def test_config5_prefill(orc, dev, qtype, N, K):
    _sampled(orc, dev, qtype, 512, N, K, seed=5, outl=0.01, rows=96)


# ------------------------------------- grouped sibling projections (pair/triple)
@pytest.mark.parametrize("qtype,M,K,Ns", [
    (Q4_K, 1, 2048, (2560, 11008)),        # 3B QKV-sized + gate-sized
    (Q4_K, 2, 2048, (11008, 11008)),       # gate + up
    (Q6_K, 1, 1024, (33, 1, 250)),         # ragged row counts
    (Q8_0, 2, 2080, (7, 129, 64)),         # K not a multiple of 256
    (Q4_K, 8, 2048, (300, 173)),           # M > 2: one MFMA launch per projection
    (Q5_K, 1, 2048, (300, 173, 64)),
    (Q4_K, 3, 2048, (300, 173)),           # activations-in-LDS GEMV, grouped
    (Q4_K, 4, 2048, (11008, 11008)),
    (Q8_K, 5, 1024, (129, 77)),
    (Q6_K, 12, 1024, (33, 1, 250)),        # slot-packed MFMA GEMV, grouped
    (Q4_K, 16, 2048, (2048, 256, 256)),
    (Q4_K, 7, 2048, (11008, 11008)),       # slot-packed GEMV, grouped wide launch
    (Q6_K, 8, 8192, (40, 64)),             # slot-packed GEMV, grouped split
    (Q4_K, 1, 5120, (5120, 1024, 1000)),   # quarter-wave rows, grouped, ragged
])
def test_grouped_parity(orc, dev, qtype, M, K, Ns):
    import torch
    from inferflux_amd import ops, synth
    note(f"grouped type={qtype} M={M} K={K} N={Ns}")
    ws = [synth.blocks(qtype, n, K, seed=11 * i + n) for i, n in enumerate(Ns)]
    x = synth.activations(M, K, seed=K + M, outlier_frac=0.01)
    a = orc.quantize_q8_1(x)
    outs = ops.qgemv_grouped(qtype, [up(w, dev) for w in ws], up(a, dev), M, list(Ns), K)
    for w, n, y in zip(ws, Ns, outs):
        check_rows(down(y), orc.gemv_exact(qtype, w, a, M, n, K))
    # accumulate mode adds onto what the outputs hold
    base = [torch.full_like(y, 0.25) for y in outs]
    ops.qgemv_grouped(qtype, [up(w, dev) for w in ws], up(a, dev), M, list(Ns), K,
                      outs=base, mode=ops.ACCUM)
    for w, n, y in zip(ws, Ns, base):
        check_rows(down(y) - 0.25, orc.gemv_exact(qtype, w, a, M, n, K))


# ---------------------- RMSNorm + Q8_1 producer fused into the grouped GEMV
@pytest.mark.parametrize("M,K,Ns,x_dtype", [
    (1, 2048, (300, 173), "f32"),        # half-wave rows (K <= 2048)
    (2, 2048, (64, 129, 200), "f16"),
    (1, 5120, (256, 77), "f32"),         # two waves per row group
    (2, 3072, (100,), "f32"),            # one wave per row group
    (1, 9216, (64, 40), "f16"),          # three waves per row group, run as four
    (2, 14336, (33,), "f32"),            # M * K/32 * 36 = 32 KB of LDS
    (1, 1280, (64,), "f32"),             # K not a multiple of 1024 (partial second pass)
    (2, 256, (40, 8, 17), "f16"),        # one super-block, three projections
])
def test_gemv_rmsnorm_fused_parity(orc, dev, M, K, Ns, x_dtype):
    """Same activations as the standalone producer (bitwise: one shared
    code path), so the fused launch equals producer + grouped GEMV bit for
    bit where the slice distribution over waves is the same, and is within
    the GEMV bar of the fp64 oracle on those activations everywhere."""
    import torch
    from inferflux_amd import ops, synth
    note(f"gemv+rmsnorm M={M} K={K} N={Ns} {x_dtype}")
    rng = np.random.default_rng(M * K + 1)
    x = (rng.standard_normal((M, K)) * 4).astype(np.float32)
    if x_dtype == "f16":
        x = x.astype(np.float16)
    nw = rng.uniform(0.2, 2.0, K).astype(np.float16)
    ws = [synth.blocks(Q4_K, n, K, seed=13 * i + n) for i, n in enumerate(Ns)]
    W = [up(w, dev) for w in ws]
    X, NW = up(x, dev), up(nw, dev)
    outs = ops.qgemv_grouped_rmsnorm(Q4_K, W, X, NW, M, list(Ns), K, eps=1e-6)
    A = ops.rmsnorm_quantize_q8_1(X, NW, eps=1e-6)
    ref = ops.qgemv_grouped(Q4_K, W, A, M, list(Ns), K)
    a = down(A)
    same_order = (K // 64 + 63) // 64 != 3  # the 3-wave row group runs as 4 waves
    for w, n, y, yr in zip(ws, Ns, outs, ref):
        y, yr = down(y), down(yr)
        if same_order:
            assert np.array_equal(y, yr), "fused launch differs from producer + GEMV"
        check_rows(y, orc.gemv_exact(Q4_K, w, a, M, n, K))
    # accumulate mode
    base = [torch.full_like(y, 0.5) for y in outs]
    ops.qgemv_grouped_rmsnorm(Q4_K, W, X, NW, M, list(Ns), K, eps=1e-6, outs=base, mode=ops.ACCUM)
    for w, n, y in zip(ws, Ns, base):
        check_rows(down(y) - 0.5, orc.gemv_exact(Q4_K, w, a, M, n, K))


@pytest.mark.parametrize("M,K,N,x_dtype", [(1, 2048, 2048, "f32"), (2, 2048, 300, "f16"),
                                           (1, 5120, 129, "f32"), (2, 4096, 64, "f16")])
def test_gemv_quantize_fused_parity(orc, dev, M, K, N, x_dtype):
    """norm_weight None: the plain quantizer fused in; bitwise equal to
    ifx_q8_1_quantize + the GEMV (same blocks, same kernel geometry)."""
    import torch
    from inferflux_amd import ops, synth
    note(f"gemv+quantize M={M} K={K} N={N} {x_dtype}")
    x = synth.activations(M, K, seed=K + M, outlier_frac=0.01)
    if x_dtype == "f16":
        x = x.astype(np.float16)
    w = synth.blocks(Q4_K, N, K, seed=N + 5)
    W, X = up(w, dev), up(x, dev)
    base = torch.full((M, N), 0.25, device=dev)
    y = ops.qgemv_grouped_rmsnorm(Q4_K, [W], X, None, M, [N], K, outs=[base.clone()],
                                  mode=ops.ACCUM)[0]
    A = ops.quantize_q8_1(X)
    yr = ops.qgemv_grouped(Q4_K, [W], A, M, [N], K, outs=[base.clone()], mode=ops.ACCUM)[0]
    assert np.array_equal(down(y), down(yr))
    a = down(A)
    assert np.array_equal(a, orc.quantize_q8_1(x.astype(np.float32)))
    check_rows(down(y) - 0.25, orc.gemv_exact(Q4_K, w, a, M, N, K))


def test_gemv_rmsnorm_fused_f16_out(orc, dev):
    """fp16 outputs of the fused launch: equal to producer + GEMV with fp16 out."""
    import torch
    from inferflux_amd import ops, synth
    M, K, Ns = 2, 2048, [96, 200]
    rng = np.random.default_rng(3)
    x = (rng.standard_normal((M, K)) * 2).astype(np.float32)
    nw = rng.uniform(0.5, 1.5, K).astype(np.float16)
    ws = [up(synth.blocks(Q4_K, n, K, seed=n), dev) for n in Ns]
    X, NW = up(x, dev), up(nw, dev)
    y = ops.qgemv_grouped_rmsnorm(Q4_K, ws, X, NW, M, Ns, K, eps=1e-5, out_dtype=torch.float16)
    A = ops.rmsnorm_quantize_q8_1(X, NW, eps=1e-5)
    yr = ops.qgemv_grouped(Q4_K, ws, A, M, Ns, K, out_dtype=torch.float16)
    for a, b in zip(y, yr):
        assert np.array_equal(down(a), down(b))


def test_gemv_rmsnorm_fused_not_handled(dev):
    import torch
    from inferflux_amd import ops
    W = torch.zeros(1 << 16, dtype=torch.uint8, device=dev)
    x = torch.zeros((4, 2048), dtype=torch.float32, device=dev)
    nw = torch.ones(2048, dtype=torch.float16, device=dev)
    for qtype, M in ((Q6_K, 1), (Q4_K, 3)):  # other types, M > 2: two calls instead
        with pytest.raises(ops.NotHandled) as e:
            ops.qgemv_grouped_rmsnorm(qtype, [W], x, nw, M, [8], 2048)
        assert e.value.status == 2


def test_host_cpp_gpu():
    """The C++ FusedQuantGemm mirror on the GPU (tests/cpp, vs the oracle)."""
    import subprocess
    from tests.test_host_cpp import binary
    note("host cpp gpu cases")
    r = subprocess.run([binary(), "gpu"], capture_output=True, text=True, timeout=100)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr


def test_host_cpp_down_proj_gpu():
    """BuildDownProjMmqLayout + DownProjMmq through the C++ mirror on the 3B
    (2048 x 11008 Q6_K, M = 1/2/4/8) and 14B (5120 x 13824 Q6_K, M = 16/32)
    down projections and Q4_K cases, against the oracle, plus the
    producer-fused extensions (tests/cpp/test_down_proj_mmq.cpp)."""
    import subprocess
    from tests.test_host_cpp import BIN_MMQ, binary
    note("host cpp down-proj mmq gpu cases")
    r = subprocess.run([binary(BIN_MMQ), "gpu"], capture_output=True, text=True, timeout=110)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr


# ------------------------------------------------ fused Q8_1 producers
def _q8_1_fields(a):
    b = a.reshape(a.shape[0], -1, 36)
    d = b[:, :, 0:2].copy().view(np.float16)[:, :, 0]
    s = b[:, :, 2:4].copy().view(np.float16)[:, :, 0]
    q = b[:, :, 4:].view(np.int8).astype(np.int32)
    return d, s, q


def check_q8_1_close(a_gpu, a_ref, y_ref):
    """The device's pre-quantization values differ from the fp64-based
    oracle's by rounding (sum order of the norm, exp, GEMV accumulation):
    codes may differ by one, rarely, and scales by one fp16 ulp; each block
    must still be a valid quantization of the reference values and its s
    field must agree with d * sum(q) of its own codes."""
    if np.array_equal(a_gpu, a_ref):
        return
    dg, sg, qg = _q8_1_fields(a_gpu)
    dr, sr, qr = _q8_1_fields(a_ref)
    diff = np.abs(qg - qr)
    assert diff.max() <= 1, f"code differs by {diff.max()}"
    # rare: at most 0.2 % of the codes (at least two for small tensors); the
    # bound below checks each code against the reference value itself
    assert (diff > 0).sum() <= max(2, 2e-3 * diff.size), f"{(diff > 0).mean():.2e} of codes differ"
    du = np.abs(dg.view(np.int16).astype(np.int32) - dr.view(np.int16).astype(np.int32))
    assert du.max() <= 1, "scale differs by more than one fp16 ulp"
    # s = f16(d * sum(q)) with the fp32 d (the block stores f16(d)): within
    # the two fp16 roundings of the stored d
    # (an s beyond the fp16 range is inf, as the format stores it)
    s_from = dg.astype(np.float64) * qg.sum(axis=2)
    big = np.abs(s_from) > 65504.0 * (1 + 2e-3)
    assert np.all(np.isinf(sg[big]))
    fin = ~big & (np.abs(s_from) < 65504.0 * (1 - 2e-3))
    assert np.all(np.abs(sg[fin].astype(np.float64) - s_from[fin]) <= 2e-3 * np.abs(s_from[fin]) + 1e-7)
    yb = y_ref.reshape(qg.shape).astype(np.float64)
    d64 = dg.astype(np.float64)[:, :, None]
    # codes come from the fp32 d; the stored fp16 d is off by up to 2^-11 d,
    # which |q| <= 127 multiplies
    bound = (0.5 + 127 * 2.0 ** -11) * d64 * (1 + 1e-3) + 1e-7 * np.abs(yb)
    assert np.all(np.abs(d64 * qg - yb) <= bound)


@pytest.mark.parametrize("x_dtype", ["f32", "f16"])
def test_rmsnorm_quantize_exact_kat(orc, dev, x_dtype):
    import torch
    from inferflux_amd import ops
    note(f"rmsnorm kat {x_dtype}")
    rng = np.random.default_rng(31)
    x = np.where(rng.random((3, 2048)) < 0.5, -1.0, 1.0).astype(np.float32)
    w = rng.standard_normal(2048).astype(np.float16)
    xt = up(x if x_dtype == "f32" else x.astype(np.float16), dev)
    a = down(ops.rmsnorm_quantize_q8_1(xt, up(w, dev), eps=0.0))
    assert np.array_equal(a, orc.rmsnorm_quantize_q8_1(x, w, 0.0))


@pytest.mark.parametrize("M,K,x_dtype", [(1, 2048, "f32"), (5, 5120, "f32"), (2, 11008, "f16"),
                                         (1, 32, "f32"), (3, 13824, "f16")])
def test_rmsnorm_quantize_parity(orc, dev, M, K, x_dtype):
    from inferflux_amd import ops
    note(f"rmsnorm M={M} K={K} {x_dtype}")
    rng = np.random.default_rng(M * K)
    x = (rng.standard_normal((M, K)) * 4).astype(np.float32)
    if x_dtype == "f16":
        x = x.astype(np.float16)
    w = rng.uniform(0.2, 2.0, K).astype(np.float16)
    a = down(ops.rmsnorm_quantize_q8_1(up(x, dev), up(w, dev), eps=1e-6))
    check_q8_1_close(a, orc.rmsnorm_quantize_q8_1(x, w, 1e-6), orc.rmsnorm_values(x, w, 1e-6))


@pytest.mark.parametrize("M,K,dtype", [(1, 11008, "f32"), (4, 13824, "f32"), (2, 2048, "f16"),
                                       (3, 32, "f32")])
def test_silu_mul_quantize_parity(orc, dev, M, K, dtype):
    from inferflux_amd import ops
    note(f"silu_mul M={M} K={K} {dtype}")
    rng = np.random.default_rng(M + K)
    g = (rng.standard_normal((M, K)) * 2).astype(np.float32)
    u = rng.standard_normal((M, K)).astype(np.float32)
    if dtype == "f16":
        g, u = g.astype(np.float16), u.astype(np.float16)
    a = down(ops.silu_mul_quantize_q8_1(up(g, dev), up(u, dev)))
    check_q8_1_close(a, orc.silu_mul_quantize_q8_1(g, u), orc.silu_mul_values(g, u))


def test_silu_mul_quantize_exact_kat(orc, dev):
    """gate >= 20: exp(-gate) vanishes in fp32 next to 1, so y = gate * up
    exactly; with integer gate/up the codes are exact on both sides."""
    from inferflux_amd import ops
    rng = np.random.default_rng(33)
    g = rng.integers(20, 40, (2, 256)).astype(np.float32)
    u = rng.integers(-3, 4, (2, 256)).astype(np.float32)
    a = down(ops.silu_mul_quantize_q8_1(up(g, dev), up(u, dev)))
    assert np.array_equal(a, orc.silu_mul_quantize_q8_1(g, u))
    assert np.array_equal(a, orc.quantize_q8_1(g * u))


# ------------------------------- fused gate/up GEMV + SiLU + Q8_1 epilogue
@pytest.mark.parametrize("qtype,M,N,K", [(Q4_K, 1, 11008, 2048), (Q4_K, 2, 1024, 2048),
                                         (Q4_K, 1, 64, 256), (Q4_K, 2, 96, 1280),
                                         (Q6_K, 1, 512, 1024), (Q8_0, 2, 64, 2080),
                                         (Q4_K, 1, 32, 5120), (Q5_K, 1, 1024, 2048),
                                         (Q8_K, 2, 512, 1024)])
def test_gate_up_silu_parity(orc, dev, qtype, M, N, K):
    import torch
    from inferflux_amd import ops, synth
    note(f"gate_up_silu type={qtype} M={M} N={N} K={K}")
    wg = synth.blocks(qtype, N, K, seed=N + 1)
    wu = synth.blocks(qtype, N, K, seed=N + 2)
    a = orc.quantize_q8_1(synth.activations(M, K, seed=K, outlier_frac=0.01))
    h, q = ops.qgemv_gate_up_silu(qtype, up(wg, dev), up(wu, dev), up(a, dev), M, N, K)
    g_ref = orc.gemv_exact(qtype, wg, a, M, N, K)
    u_ref = orc.gemv_exact(qtype, wu, a, M, N, K)
    with np.errstate(over="ignore"):
        h_ref = g_ref / (1.0 + np.exp(-g_ref)) * u_ref
    check_rows(down(h), h_ref)
    check_q8_1_close(down(q), orc.quantize_q8_1(h_ref.astype(np.float32)), h_ref)
    # fp16 h only; Q8_1 only
    h16, none = ops.qgemv_gate_up_silu(qtype, up(wg, dev), up(wu, dev), up(a, dev), M, N, K,
                                       want_q8_1=False, h_dtype=torch.float16)
    assert none is None
    h16 = down(h16).astype(np.float64)
    over = np.abs(h_ref) > 65520.0
    assert np.array_equal(h16[over], np.copysign(np.inf, h_ref[over]))
    check_rows(np.where(over, 0.0, h16), np.where(over, 0.0, h_ref), tol=2e-3)
    none, q2 = ops.qgemv_gate_up_silu(qtype, up(wg, dev), up(wu, dev), up(a, dev), M, N, K,
                                      want_h=False)
    assert none is None and np.array_equal(down(q2), down(q))


@pytest.mark.parametrize("M,N,K", [(1, 11008, 2048), (2, 1024, 2048), (1, 64, 256),
                                   (2, 96, 1280)])
def test_gate_up_silu_matches_two_launch_chain(orc, dev, M, N, K):
    """The wide Q4_K kernel (K <= 2048) computes the grouped GEMV's row sums
    in the same order and the standalone SiLU producer's arithmetic, so its
    h and Q8_1 blocks equal those of grouped GEMV + silu_mul_quantize bit for
    bit; the RMSNorm-fused variant equals RMSNorm producer + that kernel."""
    import torch
    from inferflux_amd import ops, synth
    note(f"gate_up_silu chain M={M} N={N} K={K}")
    wg = up(synth.blocks(Q4_K, N, K, seed=N + 5), dev)
    wu = up(synth.blocks(Q4_K, N, K, seed=N + 6), dev)
    rng = np.random.default_rng(K + M)
    x = torch.from_numpy(rng.standard_normal((M, K)).astype(np.float32)).to(dev)
    # norm weights small enough that h = silu(g) * u stays inside the fp16
    # range, so the fp16 comparison below compares finite values
    nw = torch.from_numpy(rng.uniform(0.05, 0.15, K).astype(np.float16)).to(dev)
    a = ops.rmsnorm_quantize_q8_1(x, nw)
    g, u = ops.qgemv_grouped(Q4_K, [wg, wu], a, M, [N, N], K)
    q_chain = down(ops.silu_mul_quantize_q8_1(g, u))
    h, q = ops.qgemv_gate_up_silu(Q4_K, wg, wu, a, M, N, K)
    gn, un = down(g).astype(np.float32), down(u).astype(np.float32)
    assert np.array_equal(down(q), q_chain)
    # device expf and the host's may differ in the last bit: h within 1e-6
    np.testing.assert_allclose(down(h), orc.silu_mul_values(gn, un), rtol=1e-6, atol=1e-30)
    for xx in (x, x.to(torch.float16)):
        a2 = ops.rmsnorm_quantize_q8_1(xx, nw)
        h2, q2 = ops.qgemv_gate_up_silu(Q4_K, wg, wu, a2, M, N, K)
        h3, q3 = ops.qgemv_gate_up_silu_rmsnorm(Q4_K, wg, wu, xx, nw, M, N, K)
        assert np.array_equal(down(q3), down(q2))
        assert np.array_equal(down(h3).view(np.uint32), down(h2).view(np.uint32))
    h16, none = ops.qgemv_gate_up_silu_rmsnorm(Q4_K, wg, wu, x, nw, M, N, K, want_q8_1=False,
                                               h_dtype=torch.float16)
    assert none is None
    assert np.isfinite(down(h16)).all()
    assert np.array_equal(down(h16), down(h).astype(np.float16))


def test_gate_up_silu_rmsnorm_not_handled(dev):
    """Not Q4_K, M > 2, N % 32 != 0 or K > 2048: not handled, nothing launched."""
    import torch
    from inferflux_amd import ops
    w = torch.zeros(1 << 22, dtype=torch.uint8, device=dev)
    x = torch.zeros(4 * 4096, dtype=torch.float32, device=dev)
    nw = torch.zeros(4096, dtype=torch.float16, device=dev)
    for qt, M, N, K in ((Q6_K, 1, 32, 256), (Q4_K, 3, 32, 256), (Q4_K, 1, 48, 256),
                        (Q4_K, 1, 32, 2304)):
        with pytest.raises(ops.NotHandled):
            ops.qgemv_gate_up_silu_rmsnorm(qt, w, w, x, nw, M, N, K)


def test_gate_up_silu_not_handled(dev):
    """M > 32, M > 2 for Q5_K (no batch kernel), N % 32 != 0, or a K split
    (fp16-dequant GEMV, M up to 32) without a workspace: not handled
    (positive status), nothing launched."""
    import torch
    from inferflux_amd import ops
    w = torch.zeros(1 << 20, dtype=torch.uint8, device=dev)
    a = torch.zeros(1 << 16, dtype=torch.uint8, device=dev)
    assert ops.gate_up_silu_workspace_bytes(Q4_K, 20, 64, 5120) > 0
    with ops.launch_log() as lg:
        for qt, M, N, K in ((Q4_K, 33, 32, 256), (Q5_K, 3, 32, 256), (Q8_0, 1, 20, 32),
                            (Q6_K, 4, 48, 256), (Q4_K, 20, 64, 5120)):
            with pytest.raises(ops.NotHandled):
                ops.qgemv_gate_up_silu(qt, w, w, a, M, N, K)
    assert lg.kernels == []


@pytest.mark.parametrize("qtype,M,N,K", [(Q4_K, 8, 11008, 2048), (Q4_K, 5, 11008, 2048),
                                         (Q4_K, 4, 11008, 2048), (Q4_K, 3, 96, 512),
                                         (Q6_K, 6, 64, 2048), (Q6_K, 8, 8192, 1024),
                                         (Q4_K, 7, 13824, 5120)])
def test_gate_up_silu_batch(orc, dev, qtype, M, N, K):
    """3 <= M <= 8 on the slot-packed MFMA GEMV with the SiLU / Q8_1
    epilogue: within the bar of the oracle, and bit for bit the grouped
    GEMV + SiLU producer wherever the grouped launch runs the same kernel."""
    import torch
    from inferflux_amd import ops, synth
    note(f"gate_up_silu batch type={qtype} M={M} N={N} K={K}")
    wg = synth.blocks(qtype, N, K, seed=N + 3)
    wu = synth.blocks(qtype, N, K, seed=N + 4)
    x = synth.activations(M, K, seed=K + M, outlier_frac=0.01) * 0.1  # h well inside fp16
    a = orc.quantize_q8_1(x)
    Wg, Wu, A = up(wg, dev), up(wu, dev), up(a, dev)
    with ops.launch_log() as lg:
        h, q = ops.qgemv_gate_up_silu(qtype, Wg, Wu, A, M, N, K)
    assert len(lg.kernels) == 1 and lg.kernels[0].startswith("k_gemv_slot<")
    idx = np.unique(np.random.default_rng(N).choice(N // 32, 24)) * 32
    idx = (idx[:, None] + np.arange(32)[None, :]).ravel()  # whole Q8_1 blocks
    g_ref = orc.gemv_exact(qtype, wg[idx], a, M, len(idx), K)
    u_ref = orc.gemv_exact(qtype, wu[idx], a, M, len(idx), K)
    h_ref = g_ref / (1.0 + np.exp(-g_ref)) * u_ref
    check_rows(down(h)[:, idx], h_ref)
    # the Q8_1 blocks are the exact quantization of the device's h
    assert np.array_equal(down(q), orc.quantize_q8_1(down(h)))
    with ops.launch_log() as lg2:
        g, u = ops.qgemv_grouped(qtype, [Wg, Wu], A, M, [N, N], K)
    if same_slot_waves(lg2.kernels[-1], lg.kernels[0]):
        assert np.array_equal(down(q), down(ops.silu_mul_quantize_q8_1(g, u)))
        np.testing.assert_allclose(down(h), orc.silu_mul_values(down(g), down(u)), rtol=1e-6,
                                   atol=1e-30)
    h16, none = ops.qgemv_gate_up_silu(qtype, Wg, Wu, A, M, N, K, want_q8_1=False,
                                       h_dtype=torch.float16)
    assert none is None
    assert np.array_equal(down(h16), down(h).astype(np.float16))


def test_gemv_only_types_not_handled(dev):
    """Q5_K / Q8_K: M > 64 and the prefill entry are not handled (the
    reference's Q8_K dispatch returns false above M = 64 and it has no fused
    Q5_K kernel): a positive status, nothing launched."""
    import torch
    from inferflux_amd import ops
    w = torch.zeros(1 << 16, dtype=torch.uint8, device=dev)
    a = torch.zeros(1 << 16, dtype=torch.uint8, device=dev)
    for qt in (Q5_K, Q8_K):
        with pytest.raises(ops.NotHandled):
            ops.qgemv(qt, w, a, 65, 8, 256)
        with pytest.raises(ops.NotHandled):
            ops.qgemv(qt, w, a, 8, 8, 256, prefill=True)
