"""The single-launch post-attention decode layer (ifx_decode_ffn) at the
Qwen2.5-3B shape: the residual it leaves equals, bit for bit, the residual
of the four-launch chain it replaces (O with the fused quantizer in
accumulate mode, gate/up + SiLU with the fused RMSNorm, down in accumulate
mode), each launch of which is parity-tested against the oracle; and the
whole layer is within the oracle bar of an fp64 restatement of the chain.
Also: repeated calls on one workspace, HIP graph capture and replay, and the
bounded barrier wait forced to expire (a tiny limit set from the host)."""
import numpy as np
import pytest

from tests.test_gpu_parity import down, note, up

pytestmark = pytest.mark.gpu

Q4_K, Q6_K = 12, 14
HIDDEN, QDIM, FFN = 2048, 2048, 11008


@pytest.fixture(scope="module")
def dev():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda:0")


@pytest.fixture(scope="module")
def layer(dev):
    from inferflux_amd import synth
    rng = np.random.default_rng(77)
    h = {
        "wo": synth.blocks(Q4_K, HIDDEN, QDIM, seed=71),
        "wg": synth.blocks(Q4_K, FFN, HIDDEN, seed=72),
        "wu": synth.blocks(Q4_K, FFN, HIDDEN, seed=73),
        "wd": synth.blocks(Q6_K, HIDDEN, FFN, seed=74),
        "attn": synth.activations(1, QDIM, seed=75),
        "resid": rng.standard_normal((1, HIDDEN)).astype(np.float32),
        # small norm weights keep silu(g) * u well inside fp32/fp16 ranges
        "nw": rng.uniform(0.05, 0.15, HIDDEN).astype(np.float16),
    }
    d = {k: up(v, dev) for k, v in h.items()}
    return h, d


def chain(d, ops, resid):
    """The four-launch chain (three launches: O, gate/up+SiLU, down)."""
    ops.qgemv_grouped_rmsnorm(Q4_K, [d["wo"]], d["attn"], None, 1, [HIDDEN], QDIM, outs=[resid],
                              mode=ops.ACCUM)
    h, hq = ops.qgemv_gate_up_silu_rmsnorm(Q4_K, d["wg"], d["wu"], resid, d["nw"], 1, FFN, HIDDEN,
                                           eps=1e-6)
    ops.qgemv(Q6_K, d["wd"], hq, 1, HIDDEN, FFN, out=resid, mode=ops.ACCUM)
    return h


def fused(d, ops, resid, ws):
    ops.decode_ffn(d["wo"], d["attn"], resid, d["nw"], d["wg"], d["wu"], d["wd"], HIDDEN, QDIM,
                   FFN, ws, eps=1e-6)


def new_ws(ops, dev):
    import torch
    n = ops.decode_ffn_workspace_bytes(1, FFN)
    assert n == 2048 + 8 * ((FFN * 4 + 255) // 256) * 256
    return torch.zeros(n, dtype=torch.uint8, device=dev)


def err_word(ws):
    return int(down(ws[8:12]).view(np.uint32)[0])


def test_decode_ffn_equals_chain(orc, layer, dev):
    from inferflux_amd import ops
    h, d = layer
    note("decode_ffn 3B vs chain")
    rc = d["resid"].clone()
    h_c = chain(d, ops, rc)
    ws = new_ws(ops, dev)
    for it in range(3):  # the workspace is left ready for the next call
        rf = d["resid"].clone()
        with ops.launch_log() as lg:
            fused(d, ops, rf, ws)
        assert lg.kernels == ["k_gemv<12,1,1,1,4,0,2,3>", "k_decode_ffn"]
        assert err_word(ws) == 0
        assert np.array_equal(down(rf).view(np.uint32), down(rc).view(np.uint32)), f"call {it}"
        cp = (FFN * 4 + 255) // 256 * 256
        for j in range(8):  # the 8 fp32 copies of h
            hj = down(ws[2048 + j * cp:2048 + j * cp + FFN * 4]).view(np.uint32)
            assert np.array_equal(hj, down(h_c).ravel().view(np.uint32))
    ctl = down(ws[0:2048]).view(np.uint32)
    assert ctl[0] == 0 and all(ctl[64 + 32 * j] == 0 for j in range(8))  # arrival counts reset
    assert ctl[1] == 3  # one barrier per call


def test_decode_ffn_oracle(orc, layer, dev):
    """fp64 restatement of the chain with the oracle's quantizers: the
    device's pre-quantization values can round differently, so each Q8_1
    code may differ by one in rare places; the bar is the contract's 1e-3 of
    the row norm of each projection's output."""
    from inferflux_amd import ops
    h, d = layer
    note("decode_ffn 3B vs oracle")
    a_o = orc.quantize_q8_1(h["attn"])
    o = orc.gemv_exact(Q4_K, h["wo"], a_o, 1, HIDDEN, QDIM)
    r1 = (h["resid"].astype(np.float64) + o).astype(np.float32)
    a = orc.rmsnorm_quantize_q8_1(r1, h["nw"], 1e-6)
    g = orc.gemv_exact(Q4_K, h["wg"], a, 1, FFN, HIDDEN)
    u = orc.gemv_exact(Q4_K, h["wu"], a, 1, FFN, HIDDEN)
    hh = g / (1.0 + np.exp(-g)) * u
    dn = orc.gemv_exact(Q6_K, h["wd"], orc.quantize_q8_1(hh.astype(np.float32)), 1, HIDDEN, FFN)
    want = r1.astype(np.float64) + dn
    rf = d["resid"].clone()
    fused(d, ops, rf, new_ws(ops, dev))
    err = np.abs(down(rf).astype(np.float64) - want).max()
    lim = 1e-3 * (np.linalg.norm(o) + np.linalg.norm(dn))
    assert err <= lim, f"{err} > {lim}"


def test_decode_ffn_graph_replay(layer, dev):
    """Captured in a HIP graph with the residual reset before it; every
    replay (with eager work in between) equals the eager call."""
    import torch
    from inferflux_amd import ops
    h, d = layer
    note("decode_ffn graph replay")
    ws = new_ws(ops, dev)
    r0 = d["resid"].clone()
    r = r0.clone()
    fused(d, ops, r, ws)
    want = down(r)
    rg = r0.clone()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        fused(d, ops, rg.copy_(r0), ws)  # warm-up on the capture stream
        torch.cuda.synchronize()
        with torch.cuda.graph(g, stream=s):
            rg.copy_(r0)
            fused(d, ops, rg, ws)
    for _ in range(3):
        g.replay()
        torch.cuda.synchronize()
        assert np.array_equal(down(rg), want)
        assert err_word(ws) == 0
        x = torch.randn(1000, device=dev) * 2  # eager work between replays
        torch.cuda.synchronize()
        del x


def test_decode_ffn_wait_limit(layer, dev):
    """A one-tick wait limit (set from the host) makes the barriers give up:
    the kernel still runs to its end and records the failure; with the
    control words zeroed again the next call is exact."""
    import torch
    from inferflux_amd import ops
    h, d = layer
    note("decode_ffn wait limit")
    ws = new_ws(ops, dev)
    ws[16:24].copy_(torch.tensor([1], dtype=torch.int64, device=dev).view(torch.uint8))
    rf = d["resid"].clone()
    fused(d, ops, rf, ws)
    torch.cuda.synchronize()
    assert err_word(ws) != 0
    ws.zero_()
    rf = d["resid"].clone()
    fused(d, ops, rf, ws)
    rc = d["resid"].clone()
    chain(d, ops, rc)
    assert err_word(ws) == 0
    assert np.array_equal(down(rf), down(rc))


def test_decode_ffn_not_handled(dev):
    """M > 1, other types, shapes beyond the kernel, a short workspace: not
    handled (positive status), nothing launched."""
    import torch
    from inferflux_amd import _lib, ops
    L = _lib.load()
    buf = torch.zeros(1 << 20, dtype=torch.uint8, device=dev)
    p = buf.data_ptr()
    nbytes = ops.decode_ffn_workspace_bytes(1, 1024)
    cases = [  # (o, gu, down types, M, q_dim, hidden, ffn, ws bytes)
        (Q4_K, Q4_K, Q6_K, 2, 256, 256, 1024, nbytes),
        (Q6_K, Q4_K, Q6_K, 1, 256, 256, 1024, nbytes),
        (Q4_K, Q4_K, Q4_K, 1, 256, 256, 1024, nbytes),
        (Q4_K, Q4_K, Q6_K, 1, 256, 2304, 1024, nbytes),
        (Q4_K, Q4_K, Q6_K, 1, 256, 256, 1024, nbytes - 1),
    ]
    for ot, gt, dt, M, q, hd, f, wsb in cases:
        with ops.launch_log() as lg:
            rc = L.ifx_decode_ffn(ot, p, p, 0, q, p, p, 1e-6, gt, p, p, f, dt, p, M, hd, p, wsb,
                                  torch.cuda.current_stream().cuda_stream)
        assert rc > 0 and lg.kernels == []


def test_decode_ffn_without_o(layer, dev):
    """W_o None: only the FFN kernel runs, on a residual that already holds
    the attention block's output; equal to the two launches after O."""
    from inferflux_amd import ops
    h, d = layer
    note("decode_ffn without O")
    rc = d["resid"].clone()
    _, hq = ops.qgemv_gate_up_silu_rmsnorm(Q4_K, d["wg"], d["wu"], rc, d["nw"], 1, FFN, HIDDEN,
                                           eps=1e-6)
    ops.qgemv(Q6_K, d["wd"], hq, 1, HIDDEN, FFN, out=rc, mode=ops.ACCUM)
    rf = d["resid"].clone()
    ws = new_ws(ops, dev)
    with ops.launch_log() as lg:
        ops.decode_ffn(None, None, rf, d["nw"], d["wg"], d["wu"], d["wd"], HIDDEN, QDIM, FFN, ws,
                       eps=1e-6)
    assert lg.kernels == ["k_decode_ffn"]
    assert np.array_equal(down(rf).view(np.uint32), down(rc).view(np.uint32))
