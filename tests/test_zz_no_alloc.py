"""The no-alloc prefill entry (ifx_qgemm_prefill_noalloc, static device
scratch as the workspace) against the entry with a caller workspace
(ifx_qgemm_prefill_ws), through the C ABI: two calls in a row, the second
with a smaller input, fp16 outputs bit for bit (no split-K atomics there),
fp32 outputs within the oracle bar; a shape beyond the scratch is refused."""
import numpy as np
import pytest

from tests.test_gpu_parity import check_rows, down, note, up

pytestmark = pytest.mark.gpu

Q4_K, Q6_K, Q8_0 = 12, 14, 8


@pytest.fixture(scope="module")
def dev():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda:0")


def test_noalloc_matches_workspace_entry(orc, dev):
    import torch
    from inferflux_amd import ops, synth
    # the second call is smaller: its workspace is a prefix of the first's
    for qtype, M, N, K in ((Q4_K, 256, 16384, 2048), (Q8_0, 128, 16400, 512)):
        note(f"noalloc type={qtype} M={M} N={N} K={K}")
        need = ops.prefill_workspace_bytes(qtype, M, N, K)
        assert 0 < need <= ops.NOALLOC_SCRATCH_BYTES
        w = synth.blocks(qtype, N, K, seed=N + M)
        a = orc.quantize_q8_1(synth.activations(M, K, seed=K + M, outlier_frac=0.01))
        W, A = up(w, dev), up(a, dev)
        ws = torch.empty(need // 2, dtype=torch.float16, device=dev)
        with ops.launch_log() as lg:
            y16 = ops.qgemm_prefill_noalloc(qtype, W, A, M, N, K, out_dtype=torch.float16)
        assert lg.kernels[0] == "k_q8_1_to_f16"  # the workspace path ran
        y16w = ops.qgemm_prefill_ws(qtype, W, A, M, N, K, ws, out_dtype=torch.float16)
        assert np.array_equal(down(y16).view(np.uint16), down(y16w).view(np.uint16))
        y = down(ops.qgemm_prefill_noalloc(qtype, W, A, M, N, K))
        idx = np.unique(np.random.default_rng(N).choice(N, 128))
        check_rows(y[:, idx], orc.gemv_exact(qtype, w[idx], a, M, len(idx), K))


def test_noalloc_refuses_beyond_scratch(dev):
    import torch
    from inferflux_amd import ops
    M, N, K = 2048, 16384, 4096  # workspace 16 MiB + 0: M * K * 2 = 16 MiB
    need = ops.prefill_workspace_bytes(Q4_K, M + 256, N, K)
    assert need > ops.NOALLOC_SCRATCH_BYTES
    W = torch.zeros(ops.weight_bytes(Q4_K, N, K), dtype=torch.uint8, device=dev)
    A = torch.zeros((M + 256) * K // 32 * 36, dtype=torch.uint8, device=dev)
    Y = torch.empty((M + 256, N), dtype=torch.float16, device=dev)
    with ops.launch_log() as lg:
        with pytest.raises(ops.NotHandled) as e:
            ops.qgemm_prefill_noalloc(Q4_K, W, A, M + 256, N, K, out=Y)
    assert e.value.status == 5 and lg.kernels == []  # IFX_SCRATCH_LIMIT, nothing launched


def test_noalloc_without_workspace_is_plain_prefill(orc, dev):
    """A shape that needs no workspace (N < 16384) runs ifx_qgemm_prefill."""
    import torch
    from inferflux_amd import ops, synth
    qtype, M, N, K = Q6_K, 200, 129, 512
    assert ops.prefill_workspace_bytes(qtype, M, N, K) == 0
    w = synth.blocks(qtype, N, K, seed=3)
    a = orc.quantize_q8_1(synth.activations(M, K, seed=4))
    W, A = up(w, dev), up(a, dev)
    y16 = ops.qgemm_prefill_noalloc(qtype, W, A, M, N, K, out_dtype=torch.float16)
    y16p = ops.qgemv(qtype, W, A, M, N, K, out_dtype=torch.float16, prefill=True)
    assert np.array_equal(down(y16).view(np.uint16), down(y16p).view(np.uint16))
