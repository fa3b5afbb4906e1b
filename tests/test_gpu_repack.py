"""The row-split repack (ifx_repack) and the M <= 2 GEMV on its layouts:
the repacked bytes against an independent numpy restatement of the layout,
and the GEMV on repacked weights against the fp64 oracle on the raw blocks
(1e-3 * ||y_row||_2) and bit for bit against the raw-layout GEMV wherever
the two launches have the same geometry."""
import numpy as np
import pytest

from tests.test_gpu_parity import check_rows, down, note, up

pytestmark = pytest.mark.gpu

Q8_0, Q6_K, Q4_K = 8, 14, 12
Q8_0_R, Q6_K_R = 108, 114


@pytest.fixture(scope="module")
def dev():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda:0")


def split_rows(qtype, w, N, K):
    """numpy restatement of the row-split layouts (include/ifx_qgemm.h)."""
    if qtype == Q8_0:
        b = w.reshape(N, K // 32, 34)
        parts = [b[:, :, 2:].reshape(N, K), b[:, :, :2].reshape(N, -1)]
    else:
        b = w.reshape(N, K // 256, 210)
        parts = [b[:, :, :128].reshape(N, -1), b[:, :, 128:192].reshape(N, -1),
                 b[:, :, 192:208].reshape(N, -1), b[:, :, 208:].reshape(N, -1)]
    row = np.concatenate(parts, axis=1)
    pad = (-row.shape[1]) % 16
    return np.concatenate([row, np.zeros((N, pad), np.uint8)], axis=1)


@pytest.mark.parametrize("qtype,N,K", [(Q8_0, 37, 2080), (Q8_0, 5, 32), (Q6_K, 17, 11008),
                                       (Q6_K, 3, 256)])
def test_repack_layout(dev, qtype, N, K):
    from inferflux_amd import ops, synth
    note(f"repack type={qtype} N={N} K={K}")
    w = synth.blocks(qtype, N, K, seed=N + K)
    W = up(w, dev)
    out = ops.repack(qtype, W, N, K)[1]
    want = split_rows(qtype, w, N, K)
    assert out.numel() == want.size == ops.weight_bytes(qtype + 100, N, K)
    assert np.array_equal(down(out).reshape(N, -1), want)


CASES = [(Q8_0, 1, 1000, 2048), (Q8_0, 2, 77, 2080), (Q8_0, 1, 3, 96),
         (Q6_K, 1, 301, 11008), (Q6_K, 2, 1000, 2048), (Q6_K, 1, 129, 5120), (Q6_K, 2, 33, 256)]


@pytest.mark.parametrize("qtype,M,N,K", CASES)
def test_gemv_row_split(orc, dev, qtype, M, N, K):
    import torch
    from inferflux_amd import ops, synth
    note(f"gemv row-split type={qtype} M={M} N={N} K={K}")
    w = synth.blocks(qtype, N, K, seed=N * 3 + K)
    a = orc.quantize_q8_1(synth.activations(M, K, seed=K + M, outlier_frac=0.01))
    W, A = up(w, dev), up(a, dev)
    rt, WR = ops.repack(qtype, W, N, K)
    ye = orc.gemv_exact(qtype, w, a, M, N, K)
    y = down(ops.qgemv(rt, WR, A, M, N, K))
    check_rows(y, ye)
    # the same launch geometry as the raw layout: the same bits
    assert np.array_equal(y.view(np.uint32), down(ops.qgemv(qtype, W, A, M, N, K)).view(np.uint32))
    rng = np.random.default_rng(N)
    base = rng.standard_normal((M, N)).astype(np.float32)
    bias = rng.standard_normal(N).astype(np.float32)
    check_rows(down(ops.qgemv(rt, WR, A, M, N, K, out=up(base, dev), mode=ops.ACCUM)), ye + base)
    check_rows(down(ops.qgemv(rt, WR, A, M, N, K, mode=ops.BIAS, bias=up(bias, dev))),
               ye + bias[None, :])
    y16 = ops.qgemv(rt, WR, A, M, N, K, out_dtype=torch.float16)
    check_rows(down(y16).astype(np.float64), ye, tol=2e-3)


def test_grouped_row_split(orc, dev):
    from inferflux_amd import ops, synth
    K, M, Ns = 1024, 1, (100, 33, 7)
    ws = [synth.blocks(Q6_K, n, K, seed=n) for n in Ns]
    a = orc.quantize_q8_1(synth.activations(M, K, seed=9))
    WR = [ops.repack(Q6_K, up(w, dev), n, K)[1] for w, n in zip(ws, Ns)]
    outs = ops.qgemv_grouped(Q6_K_R, WR, up(a, dev), M, list(Ns), K)
    for w, n, y in zip(ws, Ns, outs):
        check_rows(down(y), orc.gemv_exact(Q6_K, w, a, M, n, K))


def test_row_split_not_handled(dev):
    """Row-split weights above M = 2, on the prefill entries, or repacking a
    type without a row-split layout: not handled, nothing launched."""
    import torch
    from inferflux_amd import ops
    w = torch.zeros(1 << 20, dtype=torch.uint8, device=dev)
    a = torch.zeros(1 << 16, dtype=torch.uint8, device=dev)
    with ops.launch_log() as lg:
        for fn in (lambda: ops.qgemv(Q8_0_R, w, a, 3, 64, 256),
                   lambda: ops.qgemv(Q6_K_R, w, a, 1, 64, 256, prefill=True),
                   lambda: ops.qgemm_prefill_kernel(Q8_0_R, w, a, 64, 64, 256, ops.PREFILL_F16),
                   lambda: ops.repack(Q4_K, w, 4, 256)):
            with pytest.raises((ops.NotHandled, KeyError)):
                fn()
    assert lg.kernels == []
