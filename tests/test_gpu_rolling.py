"""The no-split form of the fp16-dequant MFMA GEMV (k_gemv_dqr), which
launches of 192 or more row groups of 128 take: each workgroup walks the
whole K of its rows, staging the activations through LDS in steps.

Checked against the fp64 oracle on sampled rows (1e-3 * ||y_row||_2) over
ragged K (a partial last stage step, a single super-block), ragged N, every
quant type on raw and tiled rows, batch sizes on both stage widths (M <= 16:
8 super-blocks a step; above, and Q8_0 at every M: 4), the store / accumulate / bias epilogues
(bit for bit against the stored result plus the base or bias), fp16 outputs
without a workspace, and the fused gate/up/SiLU form bit for bit against
the grouped launch followed by silu_mul_quantize_q8_1.  The form asks for
no workspace, ignores one given, and repeats its bits call after call; the
launches just below the row-group threshold keep the K split."""
import numpy as np
import pytest

from tests.test_gpu_parity import check_h_propagated, check_rows, down, note, up

pytestmark = pytest.mark.gpu

Q8_0, Q4_K, Q6_K = 8, 12, 14


@pytest.fixture(scope="module")
def dev():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda:0")


def weights(qtype, tiled, N, K, seed, dev):
    from inferflux_amd import ops, synth
    w = synth.blocks(qtype, N, K, seed=seed)
    if tiled:
        return w, qtype + 200, ops.repack_tiled(qtype, up(w, dev), N, K)[1]
    return w, qtype, up(w, dev)


def sample(N, seed, rows=192):
    return np.unique(np.concatenate([[0, N - 1], np.random.default_rng(seed).choice(N, rows)]))


# (quant type, tiled, M, N, K): stage steps of 4 (M > 16) or 8 super-blocks
CASES = [
    (Q4_K, True, 32, 24576, 1280),  # 5 super-blocks: one full step, one of 1
    (Q6_K, False, 24, 24600, 512),  # ragged N: the last group 24 rows
    (Q8_0, True, 20, 24576, 256),  # one super-block
    (Q8_0, False, 32, 24576, 512),
    (Q8_0, True, 12, 24576, 768),  # Q8_0: the 4-super-block stage at every M
    (Q4_K, True, 9, 24576, 2304),  # 9 super-blocks: steps of 8 and 1
    (Q4_K, True, 16, 24700, 768),
    (Q6_K, True, 32, 24576, 2048),
]


@pytest.mark.parametrize("qtype,tiled,M,N,K", CASES)
def test_rolling_gemv(orc, dev, qtype, tiled, M, N, K):
    import torch
    from inferflux_amd import ops, synth
    note(f"rolling dq type={qtype} tiled={tiled} M={M} N={N} K={K}")
    w, qt, W = weights(qtype, tiled, N, K, N + K + M, dev)
    a = orc.quantize_q8_1(synth.activations(M, K, seed=K + M, outlier_frac=0.01))
    A = up(a, dev)
    assert ops.qgemv_workspace_bytes(qt, [N], M, K) == 0
    with ops.launch_log() as lg:
        y1 = down(ops.qgemv(qt, W, A, M, N, K, out=torch.full((M, N), 7.0, device=dev)))
    wide = M > 16 or qtype == Q8_0  # the 4-super-block stage
    assert lg.kernels == [f"k_gemv_dqr<{qtype},0,{int(tiled)},0,{4 if wide else 8},"
                          f"{2 if wide else 4},8>"], lg.kernels
    idx = sample(N, M)
    ye = orc.gemv_exact(qtype, w[idx], a, M, len(idx), K)
    check_rows(y1[:, idx], ye)
    assert np.isfinite(y1).all()
    # the same bits again, with a workspace given (unused)
    ws = torch.zeros(4096, dtype=torch.uint8, device=dev)
    y2 = down(ops.qgemv(qt, W, A, M, N, K, workspace=ws))
    assert np.array_equal(y1.view(np.uint32), y2.view(np.uint32))
    assert not down(ws).any()
    rng = np.random.default_rng(N)
    base = rng.standard_normal((M, N)).astype(np.float32)
    bias = rng.standard_normal(N).astype(np.float32)
    ya = down(ops.qgemv(qt, W, A, M, N, K, out=up(base, dev), mode=ops.ACCUM))
    assert np.array_equal(ya.view(np.uint32), (y1 + base).view(np.uint32))
    yb = down(ops.qgemv(qt, W, A, M, N, K, mode=ops.BIAS, bias=up(bias, dev)))
    assert np.array_equal(yb.view(np.uint32), (y1 + bias[None, :]).view(np.uint32))
    # fp16 outputs: the fp32 sums rounded once
    y16 = down(ops.qgemv(qt, W, A, M, N, K, out_dtype=torch.float16))
    assert np.array_equal(y16, y1.astype(np.float16))


def test_rolling_grouped_and_fused(orc, dev):
    """A tiled Q4_K gate/up pair of 2 x 96 row groups at M = 17: the grouped
    launch and the fused gate/up/SiLU launch both take the no-split form,
    and the fused h and Q8_1 blocks equal grouped + silu_mul_quantize."""
    from inferflux_amd import ops, synth
    M, N, K = 17, 12288, 512
    note(f"rolling dq grouped + fused M={M} N={N} K={K}")
    wg, qt, WG = weights(Q4_K, True, N, K, 11, dev)
    wu, _, WU = weights(Q4_K, True, N, K, 12, dev)
    a = orc.quantize_q8_1(synth.activations(M, K, seed=13) * 0.1)
    A = up(a, dev)
    assert ops.gate_up_silu_workspace_bytes(qt, M, N, K) == 0
    with ops.launch_log() as lg:
        g, u = ops.qgemv_grouped(qt, [WG, WU], A, M, [N, N], K)
        h, q = ops.qgemv_gate_up_silu(qt, WG, WU, A, M, N, K)
    assert lg.kernels == ["k_gemv_dqr<12,0,1,0,4,2,8>", "k_gemv_dqr<12,0,1,1,4,2,8>"], lg.kernels
    idx = sample(N, 5)
    ge = orc.gemv_exact(Q4_K, wg[idx], a, M, len(idx), K)
    ue = orc.gemv_exact(Q4_K, wu[idx], a, M, len(idx), K)
    check_rows(down(g)[:, idx], ge)
    check_rows(down(u)[:, idx], ue)
    check_h_propagated(down(h)[:, idx], ge, ue)
    assert np.array_equal(down(q), down(ops.silu_mul_quantize_q8_1(g, u)))


@pytest.mark.parametrize("qtype,tiled,M,N,K", [(Q6_K, False, 24, 12320, 512),
                                               (Q4_K, True, 12, 12288, 768)])
def test_rolling_fused_ragged(orc, dev, qtype, tiled, M, N, K):
    """The fused form on N % 64 == 32 (the last workgroup's second half of
    outputs past N) and on the 8-super-block stage (M <= 16)."""
    from inferflux_amd import ops, synth
    note(f"rolling dq fused type={qtype} tiled={tiled} M={M} N={N} K={K}")
    wg, qt, WG = weights(qtype, tiled, N, K, 21, dev)
    wu, _, WU = weights(qtype, tiled, N, K, 22, dev)
    a = orc.quantize_q8_1(synth.activations(M, K, seed=23) * 0.1)
    A = up(a, dev)
    with ops.launch_log() as lg:
        h, q = ops.qgemv_gate_up_silu(qt, WG, WU, A, M, N, K)
    assert len(lg.kernels) == 1 and lg.kernels[0].startswith(f"k_gemv_dqr<{qtype},0,{int(tiled)},1,")
    idx = sample(N, 6)
    ge = orc.gemv_exact(qtype, wg[idx], a, M, len(idx), K)
    ue = orc.gemv_exact(qtype, wu[idx], a, M, len(idx), K)
    check_h_propagated(down(h)[:, idx], ge, ue)
    assert np.array_equal(down(q), orc.quantize_q8_1(down(h)))


def test_rolling_thresholds(dev):
    """191 row groups keep the K split; Q8_0 takes the 4-super-block stage
    at every M."""
    import torch
    from inferflux_amd import ops
    w = torch.zeros(24576 * 34 * 16, dtype=torch.uint8, device=dev)
    a = torch.zeros(32 * 16 * 36, dtype=torch.uint8, device=dev)
    with ops.launch_log() as lg:
        ops.qgemv(Q4_K, w, a, 32, 24448, 512)
        ops.qgemv(Q8_0 + 200, w, a, 16, 24576, 512)
    assert lg.kernels == ["k_fill_zero", "k_gemv_dq<12,0,1>", "k_gemv_dqr<8,0,1,0,4,2,8>"], \
        lg.kernels
