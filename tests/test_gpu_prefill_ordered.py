"""The ordered prefill (ifx_qgemm_prefill_ordered): the fp16 prefill GEMM's
K split stores each split's fp32 tile in its own workspace slot and a second
launch (k_split_sum) adds the slots in split order, instead of fp32 atomics
into a zeroed Y.  Checked against the fp64 oracle (1e-3 * ||y_row||_2), on
a workspace filled with garbage first (it needs no clearing): the same bits
on every call, accumulate and bias results bit-equal to the stored result
plus the base or bias, close to the atomic form, workspace checks, and the
config-5 Q6_K shape (six splits) on sampled output columns."""
import numpy as np
import pytest

from tests.test_gpu_parity import check_rows, down, note, up

pytestmark = pytest.mark.gpu

Q8_0, Q4_K, Q6_K = 8, 12, 14


@pytest.fixture(scope="module")
def dev():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda:0")


def garbage_ws(nbytes, dev):
    import torch
    ws = torch.empty(nbytes, dtype=torch.uint8, device=dev)
    ws.fill_(0x7F)  # 0x7F7F7F7F: a huge float wherever a slot were read unwritten
    return ws


# (quant type, M, N, K): 2-3 output tiles, so the launch splits K (8 / 4 / 2 splits)
CASES = [(Q6_K, 128, 512, 4096), (Q4_K, 128, 768, 2048), (Q8_0, 128, 300, 1024)]


@pytest.mark.parametrize("qtype,M,N,K", CASES)
def test_prefill_ordered(orc, dev, qtype, M, N, K):
    import torch
    from inferflux_amd import ops, synth
    note(f"ordered prefill type={qtype} M={M} N={N} K={K}")
    w = synth.blocks(qtype, N, K, seed=N + K)
    a = orc.quantize_q8_1(synth.activations(M, K, seed=M + K, outlier_frac=0.01))
    W, A = up(w, dev), up(a, dev)
    nb = ops.prefill_ordered_workspace_bytes(qtype, M, N, K)
    assert nb >= 2 * M * N * 4
    ws = garbage_ws(nb, dev)
    with ops.launch_log() as lg:
        y1 = down(ops.qgemm_prefill_ordered(qtype, W, A, M, N, K, ws))
    assert lg.kernels == [f"k_gemm_f16<{qtype},8,0,2,0>", "k_split_sum"], lg.kernels
    ye = orc.gemv_exact(qtype, w, a, M, N, K)
    check_rows(y1, ye)
    for _ in range(2):
        y2 = down(ops.qgemm_prefill_ordered(qtype, W, A, M, N, K, ws))
        assert np.array_equal(y1.view(np.uint32), y2.view(np.uint32))
    rng = np.random.default_rng(N)
    base = rng.standard_normal((M, N)).astype(np.float32)
    bias = rng.standard_normal(N).astype(np.float32)
    ya = down(ops.qgemm_prefill_ordered(qtype, W, A, M, N, K, ws, out=up(base, dev),
                                        mode=ops.ACCUM))
    assert np.array_equal(ya.view(np.uint32), (y1 + base).view(np.uint32))
    yb = down(ops.qgemm_prefill_ordered(qtype, W, A, M, N, K, ws, mode=ops.BIAS,
                                        bias=up(bias, dev)))
    assert np.array_equal(yb.view(np.uint32), (y1 + bias[None, :]).view(np.uint32))
    # the atomic form (plain entry) adds the same splits in another order
    with ops.launch_log() as lg:
        yt = down(ops.qgemv(qtype, W, A, M, N, K, prefill=True))
    assert lg.kernels == ["k_fill_zero", f"k_gemm_f16<{qtype},8,0,1,0>"], lg.kernels
    check_rows(yt, ye)
    assert np.abs(yt - y1).max() <= 1e-5 * np.abs(ye).max()


def test_prefill_ordered_checks(dev):
    """A workspace below the size or off the 256-byte alignment is refused
    with nothing launched; fp16 outputs (never split) and shapes that do not
    split run the workspace entry."""
    import torch
    from inferflux_amd import ops
    M, N, K = 128, 512, 4096
    w = torch.zeros(ops.weight_bytes(Q6_K, N, K), dtype=torch.uint8, device=dev)
    a = torch.zeros(M * K // 32 * 36, dtype=torch.uint8, device=dev)
    nb = ops.prefill_ordered_workspace_bytes(Q6_K, M, N, K)
    big = torch.zeros(nb + 512, dtype=torch.uint8, device=dev)
    with ops.launch_log() as lg:
        with pytest.raises(ops.NotHandled):
            ops.qgemm_prefill_ordered(Q6_K, w, a, M, N, K, big[:nb - 256])
        with pytest.raises(ops.NotHandled):
            ops.qgemm_prefill_ordered(Q6_K, w, a, M, N, K, big[16:])
    assert lg.kernels == []
    assert ops.prefill_ordered_workspace_bytes(Q6_K, M, N, K, out_dtype=torch.float16) == 0
    with ops.launch_log() as lg:
        ops.qgemm_prefill_ordered(Q6_K, w, a, M, N, K, big, out_dtype=torch.float16)
    assert lg.kernels == [f"k_gemm_f16<{Q6_K},8,1,0,0>"], lg.kernels
    # the Q4_K config-5 shape fills the GPU without a split: the fp16 copy only
    assert ops.prefill_ordered_workspace_bytes(Q4_K, 512, 27648, 5120) == \
        ops.prefill_workspace_bytes(Q4_K, 512, 27648, 5120)


def test_prefill_ordered_config5_q6k(orc, dev):
    """The config-5 down projection (Q6_K 5120 x 27648, M = 512, six splits):
    sampled output columns against the oracle, the same bits twice."""
    from inferflux_amd import ops, synth
    M, N, K = 512, 5120, 27648
    note(f"ordered prefill config 5 type={Q6_K} M={M} N={N} K={K}")
    w = synth.blocks(Q6_K, N, K, seed=4)
    x = synth.activations(M, K, seed=5, outlier_frac=0.01)
    A = ops.quantize_q8_1(up(x, dev))
    a = down(A)
    W = up(w, dev)
    ws = garbage_ws(ops.prefill_ordered_workspace_bytes(Q6_K, M, N, K), dev)
    with ops.launch_log() as lg:
        y1 = down(ops.qgemm_prefill_ordered(Q6_K, W, A, M, N, K, ws))
    assert lg.kernels == [f"k_gemm_f16<{Q6_K},8,0,2,0>", "k_split_sum"], lg.kernels
    y2 = down(ops.qgemm_prefill_ordered(Q6_K, W, A, M, N, K, ws))
    assert np.array_equal(y1.view(np.uint32), y2.view(np.uint32))
    idx = np.unique(np.concatenate([[0, N - 1], np.random.default_rng(6).choice(N, 48)]))
    ye = orc.gemv_exact(Q6_K, w[idx], a, M, len(idx), K)
    check_rows(y1[:, idx], ye)
