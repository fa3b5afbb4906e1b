"""The packed-activation path: ifx_quantize_rows_symmetric against the oracle
bit for bit (fp32 / fp16 / bf16 inputs, the reference's known answer), its
SiLU form (codes within one where exp rounds differently), and
ifx_qgemv_packed (single, pair, triple; the reference's own test shapes and
the decode shapes) against the fp64 oracle on the same codes and scales:
per output row 1e-3 * ||y_row||_2, plus the fp16 rounding of each output."""
import numpy as np
import pytest

from tests.test_gpu_parity import down, note, up

pytestmark = pytest.mark.gpu

Q8_0, Q4_K, Q6_K, Q8_K = 8, 12, 14, 15
TOL = 1e-3


@pytest.fixture(scope="module")
def dev():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from inferflux_amd import _lib
    _lib.load()  # raises if the HIP library is missing: no fallback exists
    return torch.device("cuda:0")


def _to_dtype(x, dtype, dev):
    import torch
    t = up(np.asarray(x, np.float32), dev)
    return t.to({"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16}[dtype])


@pytest.mark.parametrize("dtype", ["f32", "f16", "bf16"])
@pytest.mark.parametrize("M,K", [(2, 4), (1, 2048), (5, 5120), (3, 100), (7, 13824)])
def test_quantize_rows_symmetric_bit_exact(orc, dev, dtype, M, K):
    from inferflux_amd import ops, synth
    note(f"quantize_rows_symmetric {dtype} M={M} K={K}")
    x = _to_dtype(synth.activations(M, K, seed=M * K, outlier_frac=0.01), dtype, dev)
    codes, scales = ops.quantize_rows_symmetric(x)
    c_ref, s_ref = orc.quantize_rows_symmetric(down(x.float()))
    assert np.array_equal(down(codes), c_ref)
    assert np.array_equal(down(scales).view(np.uint32), s_ref.view(np.uint32))


@pytest.mark.parametrize("dtype", ["f32", "f16"])
def test_quantize_rows_symmetric_offset_views(orc, dev, dtype):
    """Inputs and codes at odd element offsets (views into larger buffers):
    the vector loads need 16- / 8-byte and the code stores 4-byte alignment,
    so these calls take the scalar form and still give the oracle's bits."""
    import torch
    from inferflux_amd import ops, synth
    M, K = 3, 2048
    note(f"quantize_rows_symmetric offset views {dtype}")
    x = synth.activations(M, K, seed=5, outlier_frac=0.01)
    big = _to_dtype(np.concatenate([np.zeros(1, np.float32), x.ravel()]), dtype, dev)
    xv = big[1:].view(M, K)  # one element past an aligned base
    cbig = torch.empty(M * K + 1, dtype=torch.int8, device=dev)
    cv = cbig[1:].view(M, K)
    codes, scales = ops.quantize_rows_symmetric(xv, codes=cv)
    c_ref, s_ref = orc.quantize_rows_symmetric(down(xv.float()))
    assert np.array_equal(down(codes), c_ref)
    assert np.array_equal(down(scales).view(np.uint32), s_ref.view(np.uint32))
    ubig = _to_dtype(np.concatenate([np.zeros(1, np.float32), x.ravel() * 0.5]), dtype, dev)
    codes, scales = ops.silu_mul_quantize_rows_symmetric(xv, ubig[1:].view(M, K), codes=cv)
    c2, s2 = ops.silu_mul_quantize_rows_symmetric(xv.clone(), ubig[1:].view(M, K).clone())
    assert np.array_equal(down(codes), down(c2))  # the same codes as aligned inputs
    assert np.array_equal(down(scales), down(s2))


def test_quantize_rows_symmetric_reference_kat(dev):
    """cuda_kernel::QuantizeRowsSymmetric's contract test
    (tests/unit/test_native_forward.cpp:7181-7238), fp16 input."""
    from inferflux_amd import ops
    x = _to_dtype([[-4.0, -2.0, 0.0, 4.0], [0.0, 1.5, -1.5, 3.0]], "f16", dev)
    codes, scales = ops.quantize_rows_symmetric(x)
    assert down(codes).tolist() == [[-127, -64, 0, 127], [0, 64, -64, 127]]
    assert down(scales).tolist() == [np.float32(4.0 / 127), np.float32(3.0 / 127)]


@pytest.mark.parametrize("dtype", ["f32", "f16"])
@pytest.mark.parametrize("M,K", [(1, 8), (2, 2048), (4, 11008)])
def test_silu_mul_quantize_rows_symmetric(orc, dev, dtype, M, K):
    from inferflux_amd import ops
    note(f"silu_mul_quantize_rows_symmetric {dtype} M={M} K={K}")
    rng = np.random.default_rng(M + K)
    if K == 8:  # the reference's SwiGLU quantization test (test_native_forward.cpp:7634-7700)
        g = np.array([[-1.0, 0.0, 1.0, 2.0, -2.0, 0.5, -0.5, 3.0]], np.float32)
        u = np.array([[1.0, 1.0, 1.0, 1.0, 0.5, 2.0, 4.0, 1.0]], np.float32)
    else:
        g = (rng.standard_normal((M, K)) * 2).astype(np.float32)
        u = rng.standard_normal((M, K)).astype(np.float32)
    gt, ut = _to_dtype(g, dtype, dev), _to_dtype(u, dtype, dev)
    codes, scales = ops.silu_mul_quantize_rows_symmetric(gt, ut)
    c_ref, s_ref = orc.silu_mul_quantize_rows_symmetric(down(gt.float()), down(ut.float()))
    cg, sg = down(codes).astype(np.int32), down(scales)
    if K == 8:
        assert cg.tolist() == [[-12, 0, 32, 78, -5, 28, -34, 127]]
    # exp differs from the fp64-based oracle by rounding: the row maximum, so
    # the scale, by at most a few fp32 ulps; codes by one, rarely
    assert np.all(np.abs(sg - s_ref) <= 4 * np.spacing(s_ref))
    diff = np.abs(cg - c_ref)
    assert diff.max() <= 1
    assert (diff > 0).sum() <= max(2, 2e-3 * diff.size)


def _check_f16_rows(y, ye):
    """fp16 outputs: the contract's 1e-3 * ||y_row|| plus the rounding of
    each value to fp16 (half an ulp, relative 2^-11; subnormal step 2^-24)."""
    y = np.asarray(y, np.float64)
    lim = TOL * np.linalg.norm(ye, axis=1, keepdims=True) + np.abs(ye) * 2.0 ** -11 + 2.0 ** -24
    err = np.abs(y - ye)
    assert np.all(err <= lim), f"max err {err.max()} (limit {lim[err > lim].min()})"


PACKED_CASES = [
    # the reference's pair / triple tests (test_native_forward.cpp:1508-2523)
    (Q8_0, 2, (8, 6), 32),
    (Q4_K, 2, (8, 6), 256),
    (Q4_K, 2, (8, 6, 4), 256),
    (Q6_K, 2, (8, 6), 256),
    (Q6_K, 2, (8, 6, 4), 256),
    (Q4_K, 17, (2048, 256, 256), 2048),  # its Qwen QKV long-prefill triple
    # decode shapes: config 1, the 3B down projection, wide K (full-wave rows)
    (Q4_K, 1, (11008,), 2048),
    (Q4_K, 8, (1000,), 2048),
    (Q4_K, 3, (999,), 5120),
    (Q6_K, 1, (2048,), 11008),
    (Q6_K, 5, (300, 200), 1024),
    (Q8_0, 1, (4000,), 2048),
    (Q8_0, 6, (333,), 1056),
    (Q8_K, 2, (500,), 1024),
    (Q8_K, 1, (64, 64, 64), 4096),
    # quarter-wave rows (80 slices) and 8-row column groups
    (Q4_K, 1, (13824, 13824), 5120),
    (Q6_K, 8, (500,), 5120),
    (Q4_K, 12, (300, 77), 2048),
]


@pytest.mark.parametrize("qtype,M,Ns,K", PACKED_CASES)
def test_gemv_packed_parity(orc, dev, qtype, M, Ns, K):
    from inferflux_amd import ops, synth
    note(f"gemv_packed type={qtype} M={M} N={Ns} K={K}")
    ws = [synth.blocks(qtype, n, K, seed=n + i) for i, n in enumerate(Ns)]
    x = up(synth.activations(M, K, seed=K + M, outlier_frac=0.01), dev)
    codes, scales = ops.quantize_rows_symmetric(x)
    ys = ops.qgemv_packed(qtype, [up(w, dev) for w in ws], codes, scales, M, list(Ns), K)
    c, s = down(codes), down(scales)
    for w, n, y in zip(ws, Ns, ys):
        assert y.dtype.is_floating_point and y.element_size() == 2
        _check_f16_rows(down(y).astype(np.float64), orc.gemv_packed_exact(qtype, w, c, s, M, n, K))


def test_gemv_packed_grouped_equals_single(dev):
    """A pair launch computes each projection as its single launch does."""
    from inferflux_amd import ops, synth
    K = 2048
    ws = [up(synth.blocks(Q4_K, n, K, seed=n), dev) for n in (512, 256)]
    codes, scales = ops.quantize_rows_symmetric(up(synth.activations(2, K, seed=9), dev))
    pair = ops.qgemv_packed(Q4_K, ws, codes, scales, 2, [512, 256], K)
    for w, n, y in zip(ws, (512, 256), pair):
        single = ops.qgemv_packed(Q4_K, [w], codes, scales, 2, [n], K)[0]
        assert np.array_equal(down(y).view(np.uint16), down(single).view(np.uint16))
