"""The deterministic K-split entries (ifx_qgemv_ws / ifx_qgemv_grouped_ws):
the split launches of the slot-packed and fp16-dequant MFMA GEMVs reduce
their partial sums in split order through the caller's workspace.  Checked:
the launch is the ordered-split instance with no zero fill, the result is
within the bar of the fp64 oracle, repeated calls (eager and replayed from
a HIP graph) give the same bits, and the workspace counters are zero again
after every call."""
import numpy as np
import pytest

from tests.test_gpu_parity import check_rows, down, note, up

pytestmark = pytest.mark.gpu

Q4_K, Q6_K, Q4_K_T, Q6_K_T = 12, 14, 212, 214


@pytest.fixture(scope="module")
def dev():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda:0")


def split_arg(name):
    """The SPLIT template argument of a slot (5th) or dq (3rd) launch."""
    a = name[name.index("<") + 1:-1].split(",")
    return a[4] if name.startswith("k_gemv_slot<") else a[2]


def counters_zero(ws, n_groups):
    return not down(ws[:n_groups * 4]).any()


# (qtype, M, N, K): the 3B down projection on the slot kernel (M = 4, 8),
# the 14B down on the dq kernel (M = 32, sampled rows), tiled weights
CASES = [(Q6_K, 4, 2048, 11008), (Q6_K, 8, 2048, 11008), (Q6_K, 32, 1000, 13824),
         (Q4_K, 24, 700, 5120), (Q6_K_T, 8, 2048, 11008), (Q4_K_T, 32, 600, 5120),
         (Q6_K_T, 16, 300, 13824)]


@pytest.mark.parametrize("qtype,M,N,K", CASES)
def test_ordered_split(orc, dev, qtype, M, N, K):
    import torch
    from inferflux_amd import ops, synth
    note(f"ordered split type={qtype} M={M} N={N} K={K}")
    raw = qtype % 100
    w = synth.blocks(raw, N, K, seed=N + K + M)
    a = orc.quantize_q8_1(synth.activations(M, K, seed=K + M, outlier_frac=0.01))
    W, A = up(w, dev), up(a, dev)
    if qtype > 200:
        W = ops.repack_tiled(raw, W, N, K)[1]
    nb = ops.qgemv_workspace_bytes(qtype, [N], M, K)
    assert nb > 0
    ws = torch.zeros(nb, dtype=torch.uint8, device=dev)
    with ops.launch_log() as lg:
        y1 = down(ops.qgemv(qtype, W, A, M, N, K, workspace=ws))
    assert len(lg.kernels) == 1 and split_arg(lg.kernels[0]) == "2", lg.kernels
    groups = (N + 31) // 32 if M <= 8 else (N + 127) // 128
    assert counters_zero(ws, groups)
    ye = orc.gemv_exact(raw, w, a, M, N, K)
    check_rows(y1, ye)
    for _ in range(3):
        y2 = down(ops.qgemv(qtype, W, A, M, N, K, workspace=ws))
        assert np.array_equal(y1.view(np.uint32), y2.view(np.uint32))
    assert counters_zero(ws, groups)
    # epilogues: accumulate and bias on the ordered path
    rng = np.random.default_rng(N)
    base = rng.standard_normal((M, N)).astype(np.float32)
    bias = rng.standard_normal(N).astype(np.float32)
    ya = down(ops.qgemv(qtype, W, A, M, N, K, out=up(base, dev), mode=ops.ACCUM, workspace=ws))
    check_rows(ya, ye + base)
    assert np.array_equal(ya.view(np.uint32), (y1 + base).view(np.uint32))
    yb = down(ops.qgemv(qtype, W, A, M, N, K, mode=ops.BIAS, bias=up(bias, dev), workspace=ws))
    assert np.array_equal(yb.view(np.uint32), (y1 + bias[None, :]).view(np.uint32))
    assert counters_zero(ws, groups)


def test_ordered_split_grouped_and_graph(orc, dev):
    """Q/K/V-shaped siblings at M = 32 on the ordered dq split, captured in
    a HIP graph: every replay equals the eager result bit for bit."""
    import torch
    from inferflux_amd import ops, synth
    M, K, Ns = 32, 5120, (512, 128, 128)
    ws_ = [synth.blocks(Q4_K, n, K, seed=n) for n in Ns]
    a = orc.quantize_q8_1(synth.activations(M, K, seed=5))
    Ws, A = [up(w, dev) for w in ws_], up(a, dev)
    nb = ops.qgemv_workspace_bytes(Q4_K, list(Ns), M, K)
    ws = torch.zeros(nb, dtype=torch.uint8, device=dev)
    with ops.launch_log() as lg:
        ref = [down(y) for y in ops.qgemv_grouped(Q4_K, Ws, A, M, list(Ns), K, workspace=ws)]
    assert len(lg.kernels) == 1 and split_arg(lg.kernels[0]) == "2", lg.kernels
    for w, n, y in zip(ws_, Ns, ref):
        check_rows(y, orc.gemv_exact(Q4_K, w, a, M, n, K))
    outs = [torch.empty(M, n, device=dev) for n in Ns]
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        ops.qgemv_grouped(Q4_K, Ws, A, M, list(Ns), K, outs=outs, workspace=ws)
    for _ in range(4):
        for o in outs:
            o.fill_(7.0)
        g.replay()
        torch.cuda.synchronize()
        for o, r in zip(outs, ref):
            assert np.array_equal(down(o).view(np.uint32), r.view(np.uint32))
    assert not down(ws[:4 * 64]).any()


def test_ordered_split_workspace_checks(dev):
    """A workspace below the size or off the 256-byte alignment is refused
    with nothing launched; launches that do not split ignore it."""
    import torch
    from inferflux_amd import ops
    w = torch.zeros(1 << 25, dtype=torch.uint8, device=dev)
    a = torch.zeros(1 << 20, dtype=torch.uint8, device=dev)
    nb = ops.qgemv_workspace_bytes(Q6_K, [2048], 8, 11008)
    small = torch.zeros(nb - 256, dtype=torch.uint8, device=dev)
    big = torch.zeros(nb + 512, dtype=torch.uint8, device=dev)
    with ops.launch_log() as lg:
        with pytest.raises(ops.NotHandled):
            ops.qgemv(Q6_K, w, a, 8, 2048, 11008, workspace=small)
        with pytest.raises(ops.NotHandled):
            ops.qgemv(Q6_K, w, a, 8, 2048, 11008, workspace=big[16:])
    assert lg.kernels == []
    assert ops.qgemv_workspace_bytes(Q4_K, [11008], 1, 2048) == 0  # the M = 1 GEMV
    with ops.launch_log() as lg:
        ops.qgemv(Q4_K, w, a, 1, 2048, 2048, workspace=small)
    assert len(lg.kernels) == 1
