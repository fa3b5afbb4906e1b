"""The tiled repack (ifx_repack_tiled) and the MFMA batch GEMVs on its
layouts: the tiled bytes against an independent numpy restatement of the
layout, the GEMVs on tiled weights against the fp64 oracle on the raw blocks
(1e-3 * ||y_row||_2), and bit for bit against the raw-layout launch wherever
the dispatch runs the same kernel and split on both."""
import numpy as np
import pytest

from tests.test_gpu_parity import (check_h_propagated, check_q8_1_close, check_rows, down, note,
                                   same_slot_waves, up)

pytestmark = pytest.mark.gpu

Q8_0, Q4_K, Q6_K = 8, 12, 14
Q8_0_T, Q4_K_T, Q6_K_T = 208, 212, 214


@pytest.fixture(scope="module")
def dev():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda:0")


def tile_rows(qtype, w, N, K):
    """numpy restatement of the tiled layouts (include/ifx_qgemm.h): per
    group of 32 rows and super-block, the rows' 16-byte pieces in lane
    order (piece j of row c at 512 j + 16 c for the K-half-major pieces)."""
    nb = {Q4_K: 144, Q6_K: 210, Q8_0: 272}[qtype]  # bytes per row and 256 values
    nsb = K // 256
    G = (N + 31) // 32
    b = np.zeros((G * 32, nsb, nb), np.uint8)
    b[:N] = w.reshape(N, nsb, nb)
    b = b.reshape(G, 32, nsb, nb).transpose(0, 2, 1, 3)  # [group][sb][row][bytes]
    if qtype == Q8_0:
        blk = b.reshape(G, nsb, 32, 8, 34)
        codes = blk[..., 2:].reshape(G, nsb, 32, 8, 2, 16).transpose(0, 1, 3, 4, 2, 5)  # [j][h][row]
        d = blk[..., :2].reshape(G, nsb, 32 * 16)
        tile = np.concatenate([codes.reshape(G, nsb, 8192), d], axis=2)
    elif qtype == Q4_K:
        hdr = b[:, :, :, :16].reshape(G, nsb, 512)
        qs = b[:, :, :, 16:].reshape(G, nsb, 32, 8, 16).transpose(0, 1, 3, 2, 4)  # [p*2+h][row]
        tile = np.concatenate([hdr, qs.reshape(G, nsb, 4096)], axis=2)
    else:
        q = b[:, :, :, :192].reshape(G, nsb, 32, 12, 16).transpose(0, 1, 3, 2, 4)
        sc = b[:, :, :, 192:208].reshape(G, nsb, 512)
        d = b[:, :, :, 208:].reshape(G, nsb, 64)
        tile = np.concatenate([q.reshape(G, nsb, 6144), sc, d], axis=2)
    return tile.reshape(-1)


def _args(name):
    return name[:name.index("<")], name[name.index("<") + 1:-1].split(",")


def raw_launch(tiled_name):
    """The launch-log name of the same kernel on raw rows: the template
    arguments before the layout flag (slot: 5, dq: 3)."""
    k, a = _args(tiled_name)
    return f"{k}<{','.join(a[:5] if k == 'k_gemv_slot' else a[:3])}>"


def atomic(name):
    """A K split with fp32 atomics (its bits vary run to run)."""
    k, a = _args(name)
    return a[4 if k == "k_gemv_slot" else 2] == "1"


@pytest.mark.parametrize("qtype,N,K", [(Q4_K, 64, 512), (Q4_K, 100, 2048), (Q6_K, 33, 256),
                                       (Q6_K, 2048, 1024), (Q8_0, 70, 512)])
def test_tiled_layout(dev, qtype, N, K):
    from inferflux_amd import ops, synth
    note(f"tiled layout type={qtype} N={N} K={K}")
    w = synth.blocks(qtype, N, K, seed=N + K)
    tt, out = ops.repack_tiled(qtype, up(w, dev), N, K)
    want = tile_rows(qtype, w, N, K)
    assert tt == qtype + 200
    assert out.numel() == want.size == ops.weight_bytes(tt, N, K)
    assert np.array_equal(down(out), want)


CASES = [(Q4_K, M, 1000, 2048) for M in (1, 2, 3, 5, 8, 9, 16, 17, 32)]
CASES += [(Q6_K, M, 1000, 2048) for M in (1, 4, 8, 12, 32)]
CASES += [(Q4_K, 8, 100, 5120), (Q6_K, 5, 77, 11008), (Q6_K, 32, 2048, 5120), (Q4_K, 24, 31, 256)]
CASES += [(Q8_0, M, 1000, 2048) for M in (1, 4, 8, 12, 24, 32)] + [(Q8_0, 8, 40, 11008)]


@pytest.mark.parametrize("qtype,M,N,K", CASES)
def test_gemv_tiled(orc, dev, qtype, M, N, K):
    import torch
    from inferflux_amd import ops, synth
    note(f"gemv tiled type={qtype} M={M} N={N} K={K}")
    w = synth.blocks(qtype, N, K, seed=N * 5 + K + M)
    a = orc.quantize_q8_1(synth.activations(M, K, seed=K + M, outlier_frac=0.01))
    W, A = up(w, dev), up(a, dev)
    tt, WT = ops.repack_tiled(qtype, W, N, K)
    ye = orc.gemv_exact(qtype, w, a, M, N, K)
    with ops.launch_log() as lg:
        y = down(ops.qgemv(tt, WT, A, M, N, K))
    fam = "k_gemv_slot<" if M <= 16 else "k_gemv_dq<"  # N < 8192 here
    assert len(lg.kernels) >= 1 and lg.kernels[-1].startswith(fam) and lg.kernels[-1].endswith(",1>")
    check_rows(y, ye)
    # the raw layout on the same kernel (same arguments but the layout flag)
    # and without a K split: the same bits
    with ops.launch_log() as lr:
        yr = down(ops.qgemv(qtype, W, A, M, N, K))
    if lr.kernels[-1] == raw_launch(lg.kernels[-1]) and not atomic(lr.kernels[-1]):
        assert np.array_equal(y.view(np.uint32), yr.view(np.uint32))
    rng = np.random.default_rng(N + M)
    base = rng.standard_normal((M, N)).astype(np.float32)
    bias = rng.standard_normal(N).astype(np.float32)
    check_rows(down(ops.qgemv(tt, WT, A, M, N, K, out=up(base, dev), mode=ops.ACCUM)), ye + base)
    check_rows(down(ops.qgemv(tt, WT, A, M, N, K, mode=ops.BIAS, bias=up(bias, dev))),
               ye + bias[None, :])
    try:  # fp16 outputs above M = 8 only where K fits one activation stage
        y16 = ops.qgemv(tt, WT, A, M, N, K, out_dtype=torch.float16)
    except ops.NotHandled:
        assert M > 8
    else:
        check_rows(down(y16).astype(np.float64), ye, tol=2e-3)


@pytest.mark.parametrize("M", [1, 4, 8, 16, 32])
def test_grouped_tiled(orc, dev, M):
    """Q/K/V-shaped siblings (ragged N) in one launch."""
    from inferflux_amd import ops, synth
    note(f"grouped tiled M={M}")
    K, Ns = 1024, (300, 70, 70)
    ws = [synth.blocks(Q4_K, n, K, seed=n + M) for n in Ns]
    a = orc.quantize_q8_1(synth.activations(M, K, seed=9 + M))
    WT = [ops.repack_tiled(Q4_K, up(w, dev), n, K)[1] for w, n in zip(ws, Ns)]
    outs = ops.qgemv_grouped(Q4_K_T, WT, up(a, dev), M, list(Ns), K)
    for w, n, y in zip(ws, Ns, outs):
        check_rows(down(y), orc.gemv_exact(Q4_K, w, a, M, n, K))


@pytest.mark.parametrize("qtype,M", [(Q4_K, 1), (Q4_K, 4), (Q4_K, 8), (Q6_K, 3), (Q4_K, 12),
                                     (Q4_K, 16), (Q6_K, 9)])
def test_gate_up_silu_tiled(orc, dev, qtype, M):
    from inferflux_amd import ops, synth
    note(f"gate_up_silu tiled type={qtype} M={M}")
    N, K = 512, 1024
    wg = synth.blocks(qtype, N, K, seed=M + 1)
    wu = synth.blocks(qtype, N, K, seed=M + 2)
    x = synth.activations(M, K, seed=K + M) * 0.1
    a = orc.quantize_q8_1(x)
    A = up(a, dev)
    tt, WG = ops.repack_tiled(qtype, up(wg, dev), N, K)
    WU = ops.repack_tiled(qtype, up(wu, dev), N, K)[1]
    with ops.launch_log() as lg:
        h, q = ops.qgemv_gate_up_silu(tt, WG, WU, A, M, N, K)
    assert len(lg.kernels) == 1 and lg.kernels[0].endswith(",1,1>")
    g = orc.gemv_exact(qtype, wg, a, M, N, K)
    u = orc.gemv_exact(qtype, wu, a, M, N, K)
    check_rows(down(h), g / (1.0 + np.exp(-g)) * u)
    assert np.array_equal(down(q), orc.quantize_q8_1(down(h)))
    if 3 <= M <= 8:  # the raw layout runs the same kernel: the same bits
        hr, qr = ops.qgemv_gate_up_silu(qtype, up(wg, dev), up(wu, dev), A, M, N, K)
        assert np.array_equal(down(h).view(np.uint32), down(hr).view(np.uint32))
        assert np.array_equal(down(q), down(qr))
    if M > 8:  # 16-row slots: grouped GEMV + SiLU producer on the same geometry
        assert lg.kernels[0].startswith(f"k_gemv_slot<{qtype},16,")
        with ops.launch_log() as lg2:
            g2, u2 = ops.qgemv_grouped(tt, [WG, WU], A, M, [N, N], K)
        if same_slot_waves(lg2.kernels[-1], lg.kernels[0]):
            assert np.array_equal(down(q), down(ops.silu_mul_quantize_q8_1(g2, u2)))


@pytest.mark.parametrize("qtype,tiled,M,N,K", [(Q4_K, True, 17, 512, 1024), (Q4_K, True, 32, 1056, 5120),
                                                (Q6_K, True, 24, 512, 2048), (Q4_K, False, 32, 512, 5120),
                                                (Q8_0, False, 20, 256, 2048), (Q4_K, False, 12, 256, 2048)])
def test_gate_up_silu_dq(orc, dev, qtype, tiled, M, N, K):
    """M up to 32: the fp16-dequant GEMV with the SiLU / Q8_1 epilogue,
    through the workspace entry when its K splits.  h against the oracle,
    its Q8_1 blocks the exact quantization of h, and bit for bit the grouped
    (workspace) launch + SiLU producer where that launch is the same GEMV."""
    import torch
    from inferflux_amd import ops, synth
    note(f"gate_up_silu dq type={qtype} tiled={tiled} M={M} N={N} K={K}")
    wg = synth.blocks(qtype, N, K, seed=M + 3)
    wu = synth.blocks(qtype, N, K, seed=M + 4)
    a = orc.quantize_q8_1(synth.activations(M, K, seed=K + M) * 0.1)
    A = up(a, dev)
    if tiled:
        tt, WG = ops.repack_tiled(qtype, up(wg, dev), N, K)
        WU = ops.repack_tiled(qtype, up(wu, dev), N, K)[1]
    else:
        tt, WG, WU = qtype, up(wg, dev), up(wu, dev)
    nb = ops.gate_up_silu_workspace_bytes(tt, M, N, K)
    ws = torch.zeros(max(nb, 256), dtype=torch.uint8, device=dev)
    for rep in range(2):  # the second call reuses the workspace the first left zeroed
        with ops.launch_log() as lg:
            h, q = ops.qgemv_gate_up_silu(tt, WG, WU, A, M, N, K, workspace=ws)
        assert len(lg.kernels) == 1 and lg.kernels[0].startswith(f"k_gemv_dq<{qtype},0,")
        assert lg.kernels[0].endswith(f",{int(tiled)},1>")
        g = orc.gemv_exact(qtype, wg, a, M, N, K)
        u = orc.gemv_exact(qtype, wu, a, M, N, K)
        check_h_propagated(down(h), g, u)
        assert np.array_equal(down(q), orc.quantize_q8_1(down(h)))
    nbg = ops.qgemv_workspace_bytes(tt, [N, N], M, K)
    wsg = torch.zeros(max(nbg, 256), dtype=torch.uint8, device=dev)
    with ops.launch_log() as lg2:
        g2, u2 = ops.qgemv_grouped(tt, [WG, WU], A, M, [N, N], K, workspace=wsg)
    if lg2.kernels[-1].startswith("k_gemv_dq<"):
        assert np.array_equal(down(q), down(ops.silu_mul_quantize_q8_1(g2, u2)))
    if nb:  # without the workspace the split launch is not handled
        with pytest.raises(ops.NotHandled):
            ops.qgemv_gate_up_silu(tt, WG, WU, A, M, N, K)


def test_tiled_not_handled(dev):
    """Tiled weights above M = 32, on the prefill, fused-RMSNorm and
    dequantize entries, or tiling a type without a tiled layout: not
    handled, nothing launched (Q5_K has no tiled layout)."""
    import torch
    from inferflux_amd import ops
    w = torch.zeros(1 << 20, dtype=torch.uint8, device=dev)
    a = torch.zeros(1 << 18, dtype=torch.uint8, device=dev)
    x = torch.zeros(64, 256, device=dev)
    nw = torch.ones(256, dtype=torch.float16, device=dev)
    with ops.launch_log() as lg:
        for fn in (lambda: ops.qgemv(Q4_K_T, w, a, 33, 64, 256),
                   lambda: ops.qgemv(Q6_K_T, w, a, 1, 64, 256, prefill=True),
                   lambda: ops.qgemm_prefill_kernel(Q4_K_T, w, a, 64, 64, 256, ops.PREFILL_F16),
                   lambda: ops.qgemv_grouped_rmsnorm(Q4_K_T, [w], x[:1], nw, 1, [64], 256),
                   lambda: ops.dequantize(Q4_K_T, w, 64, 256),
                   lambda: ops.repack_tiled(13, w, 4, 256)):
            with pytest.raises((ops.NotHandled, KeyError)):
                fn()
    assert lg.kernels == []
