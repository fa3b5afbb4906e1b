"""Every launch the benchmark times, run on the GPU at its production shape
(tests/launch_table.py): the launch log must show the kernel instance the
table names, and the outputs must pass the oracle bar (1e-3 * ||y_row||_2
against the fp64 oracle) on sampled weight rows.  The fused-producer
launches are also compared bit for bit with the producer + GEMV chain they
replace."""
import numpy as np
import pytest

from tests.launch_table import IDS, LAUNCHES
from tests.test_gpu_parity import (check_h_propagated, check_q8_1_close, check_rows, down, note,
                                   same_slot_waves, up)

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda:0")


def _rows(N, seed, n=256):
    return np.unique(np.concatenate([[0, N - 1], np.random.default_rng(seed).choice(N, n)]))


@pytest.mark.parametrize("lid,entry,qt,M,Ns,K,want", LAUNCHES, ids=IDS)
def test_bench_launch(orc, dev, lid, entry, qt, M, Ns, K, want):
    import torch
    from inferflux_amd import ops, synth
    note(f"launch {lid}: {entry} type={qt} M={M} N={Ns} K={K} -> {want}")
    seed = sum(Ns) + K + M
    # row-split / tiled types: repack raw blocks on the GPU
    raw_qt = qt % 100 if qt > 100 else qt

    def to_dev(w, n):
        if entry.startswith("mmq"):
            return ops.mmq_layout(qt, up(w, dev), n, K)
        if qt > 200:
            return ops.repack_tiled(raw_qt, up(w, dev), n, K)[1]
        if qt > 100:
            return ops.repack(raw_qt, up(w, dev), n, K)[1]
        return up(w, dev)
    ws = [synth.blocks(raw_qt, n, K, seed=seed + i) for i, n in enumerate(Ns)]
    W = [to_dev(w, n) for w, n in zip(ws, Ns)]
    # the _ws entries: a zeroed workspace of the size the launch asks for
    wsp = None
    if entry.endswith("_ws"):
        entry = entry[:-3]
        nb = (ops.gate_up_silu_workspace_bytes(qt, M, Ns[0], K) if entry == "gate_up_silu"
              else 0 if entry == "mmq_accum"  # the layout's own
              else ops.qgemv_workspace_bytes(qt, list(Ns), M, K))
        wsp = torch.zeros(max(nb, 256), dtype=torch.uint8, device=dev)
    rng = np.random.default_rng(seed)
    outl = 0.01 if entry.startswith("prefill") else 0.0
    x = synth.activations(M, K, seed=seed + 7, outlier_frac=outl)
    base = rng.standard_normal((M, max(Ns))).astype(np.float32)

    if entry in ("grouped_rmsnorm", "gate_up_silu_rmsnorm"):
        nw = rng.uniform(0.5, 1.5, K).astype(np.float16)
        X, NW = up(x, dev), up(nw, dev)
        A = ops.rmsnorm_quantize_q8_1(X, NW, eps=1e-6)  # the standalone producer
        a = down(A)
        check_q8_1_close(a, orc.rmsnorm_quantize_q8_1(x, nw, 1e-6), orc.rmsnorm_values(x, nw, 1e-6))
    elif entry == "packed":
        X = up(x, dev)
        codes, scales = ops.quantize_rows_symmetric(X)
        c_h, s_h = down(codes), down(scales)
        assert np.array_equal(c_h, orc.quantize_rows_symmetric(x)[0])
    else:
        a = orc.quantize_q8_1(x)
        A = up(a, dev)
        X = up(x, dev)

    if entry.startswith("gate_up_silu"):
        wu = synth.blocks(raw_qt, Ns[0], K, seed=seed + 11)
        Wu = to_dev(wu, Ns[0])
    with ops.launch_log() as lg:
        if entry == "gemv":
            outs = [ops.qgemv(qt, W[0], A, M, Ns[0], K, workspace=wsp)]
        elif entry in ("gemv_accum", "quantize_accum", "mmq_accum"):
            y0 = up(base[:, :Ns[0]], dev)
            if entry == "mmq_accum":
                ops.qgemv_mmq(qt, W[0], A, M, Ns[0], K, out=y0, mode=ops.ACCUM,
                              ordered=wsp is not None)
            elif entry == "gemv_accum":
                ops.qgemv(qt, W[0], A, M, Ns[0], K, out=y0, mode=ops.ACCUM, workspace=wsp)
            else:
                ops.qgemv_grouped_rmsnorm(qt, W, X, None, M, list(Ns), K, outs=[y0],
                                          mode=ops.ACCUM)
            outs = [y0]
        elif entry == "grouped":
            outs = ops.qgemv_grouped(qt, W, A, M, list(Ns), K, workspace=wsp)
        elif entry == "grouped_rmsnorm":
            outs = ops.qgemv_grouped_rmsnorm(qt, W, X, NW, M, list(Ns), K, eps=1e-6)
        elif entry == "gate_up_silu_rmsnorm":
            h, q = ops.qgemv_gate_up_silu_rmsnorm(qt, W[0], Wu, X, NW, M, Ns[0], K, eps=1e-6)
        elif entry == "gate_up_silu":
            h, q = ops.qgemv_gate_up_silu(qt, W[0], Wu, A, M, Ns[0], K, workspace=wsp)
        elif entry == "packed":
            outs = ops.qgemv_packed(qt, W, codes, scales, M, list(Ns), K)
        elif entry == "prefill":
            outs = [ops.qgemv(qt, W[0], A, M, Ns[0], K, prefill=True)]
        elif entry == "prefill_int8":
            outs = [ops.qgemm_prefill_kernel(qt, W[0], A, M, Ns[0], K, ops.PREFILL_INT8)]
        else:
            raise ValueError(entry)
        torch.cuda.synchronize()
    assert lg.kernels == want

    if entry in ("gate_up_silu_rmsnorm", "gate_up_silu"):
        N = Ns[0]
        blocks = np.random.default_rng(seed).choice(N // 32, 16, replace=False)
        idx = (blocks[:, None] * 32 + np.arange(32)[None, :]).ravel()
        g = orc.gemv_exact(raw_qt, ws[0][idx], a, M, len(idx), K)
        u = orc.gemv_exact(raw_qt, wu[idx], a, M, len(idx), K)
        with np.errstate(over="ignore"):
            h_ref = g / (1.0 + np.exp(-g)) * u
        if want[0].startswith("k_gemv_dq<"):  # fp16 weights: the GEMV bar carried through h
            check_h_propagated(down(h)[:, idx], g, u)
        else:
            check_rows(down(h)[:, idx], h_ref)
        # the Q8_1 blocks are the exact quantization of the device's h
        assert np.array_equal(down(q), orc.quantize_q8_1(down(h)))
        # the chain it replaces: grouped GEMV + SiLU producer, bit for bit
        # where the grouped launch forms the sums in the same order
        wsg = None
        if wsp is not None:
            nbg = ops.qgemv_workspace_bytes(qt, [N, N], M, K)
            wsg = torch.zeros(max(nbg, 256), dtype=torch.uint8, device=dev)
        with ops.launch_log() as lg2:
            g2, u2 = ops.qgemv_grouped(qt, [W[0], Wu], A, M, [N, N], K, workspace=wsg)
        same_dq = lg2.kernels[-1].startswith("k_gemv_dq<") and want[0].startswith("k_gemv_dq<")
        if entry == "gate_up_silu_rmsnorm" or same_dq or same_slot_waves(lg2.kernels[-1], want[0]):
            assert np.array_equal(down(q), down(ops.silu_mul_quantize_q8_1(g2, u2)))
        return

    if entry == "packed":
        # fp16 outputs: the row bar plus each value's fp16 rounding
        for i, (w, n, y) in enumerate(zip(ws, Ns, outs)):
            idx = _rows(n, seed + i)
            ye = orc.gemv_packed_exact(raw_qt, w[idx], c_h, s_h, M, len(idx), K)
            yd = down(y)[:, idx].astype(np.float64)
            lim = 1e-3 * np.linalg.norm(ye, axis=1, keepdims=True) + np.abs(ye) * 2.0 ** -11
            assert np.all(np.abs(yd - ye) <= lim)
        return

    for i, (w, n, y) in enumerate(zip(ws, Ns, outs)):
        idx = _rows(n, seed + i)
        ye = orc.gemv_exact(raw_qt, w[idx], a, M, len(idx), K)
        if entry in ("gemv_accum", "quantize_accum", "mmq_accum"):
            ye = ye + base[:, idx]
        yd = down(y)
        assert np.isfinite(yd).all()
        check_rows(yd[:, idx], ye)
    if entry == "grouped_rmsnorm":
        # bit for bit the standalone producer + grouped GEMV (same geometry)
        ref = ops.qgemv_grouped(qt, W, A, M, list(Ns), K)
        for y, yr in zip(outs, ref):
            assert np.array_equal(down(y), down(yr))
