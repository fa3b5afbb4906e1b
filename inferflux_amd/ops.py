"""Torch-facing wrappers over the C ABI (include/ifx_qgemm.h).

PyTorch only provides device memory and the current HIP stream here; every
computation is a HIP kernel in libifx_qgemm.so, called through ctypes.
Errors follow the reference's contract (fused_quant_gemm.cu:2085-2117):
a positive status means "not handled" and is raised as NotHandled so the
caller can pick a fallback; a negative status is a HIP launch error.
"""

import torch

from . import _lib

Q8_0, Q8_1, Q4_K, Q5_K, Q6_K, Q8_K = 8, 9, 12, 13, 14, 15
Q8_0_R, Q6_K_R = 108, 114  # row-split layouts written by repack()
Q8_0_T, Q4_K_T, Q6_K_T = 208, 212, 214  # tiled layouts written by repack_tiled()
BLOCK_BYTES = {Q4_K: 144, Q5_K: 176, Q6_K: 210, Q8_0: 34, Q8_1: 36, Q8_K: 292}
BLOCK_ELEMS = {Q4_K: 256, Q5_K: 256, Q6_K: 256, Q8_0: 32, Q8_1: 32, Q8_K: 256}
TYPE_NAMES = {Q4_K: "Q4_K", Q5_K: "Q5_K", Q6_K: "Q6_K", Q8_0: "Q8_0", Q8_1: "Q8_1", Q8_K: "Q8_K",
              108: "Q8_0_R", 114: "Q6_K_R", 208: "Q8_0_T", 212: "Q4_K_T", 214: "Q6_K_T"}

STORE, ACCUM, BIAS = 0, 1, 2
OUT_F32, OUT_F16 = 0, 1


class NotHandled(RuntimeError):
    """Positive status: the call launched nothing (reference: `false`)."""

    def __init__(self, status, what):
        super().__init__(f"{what}: {_lib.load().ifx_status_string(status).decode()} ({status})")
        self.status = status


class HipError(RuntimeError):
    pass


def _check(rc, what):
    if rc == 0:
        return
    if rc > 0:
        raise NotHandled(rc, what)
    raise HipError(f"{what}: HIP error {-rc}: {_lib.load().ifx_status_string(rc).decode()}")


def _stream(stream):
    if stream is None:
        stream = torch.cuda.current_stream()
    return stream.cuda_stream


def _dev(t, name):
    if not t.is_cuda:
        raise ValueError(f"{name} must be a device tensor")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")
    return t.data_ptr()


def weight_bytes(qtype, n_rows, K):
    if qtype in (Q8_0_R, Q6_K_R):
        return n_rows * _row_split_bytes(qtype, K)
    if qtype in (Q8_0_T, Q4_K_T, Q6_K_T):  # whole groups of 32 rows
        raw = qtype - 200
        return (n_rows + 31) // 32 * 32 * (K // BLOCK_ELEMS[raw]) * BLOCK_BYTES[raw]
    return n_rows * (K // BLOCK_ELEMS[qtype]) * BLOCK_BYTES[qtype]


def quantize_q8_1(x, out=None, stream=None):
    """fp32 or fp16 x [M, K] (device) -> uint8 Q8_1 blocks [M, K/32*36]."""
    M, K = x.shape
    if out is None:
        out = torch.empty((M, K // 32 * 36), dtype=torch.uint8, device=x.device)
    L = _lib.load()
    if x.dtype == torch.float32:
        rc = L.ifx_q8_1_quantize_f32(_dev(x, "x"), _dev(out, "out"), M, K, _stream(stream))
    elif x.dtype == torch.float16:
        rc = L.ifx_q8_1_quantize_f16(_dev(x, "x"), _dev(out, "out"), M, K, _stream(stream))
    else:
        raise TypeError("x must be float32 or float16")
    _check(rc, "ifx_q8_1_quantize")
    return out


def rmsnorm_quantize_q8_1(x, norm_weight, eps=1e-6, out=None, stream=None):
    """RMSNorm of fp32/fp16 rows x [M, K] by fp16 norm_weight [K], then Q8_1."""
    M, K = x.shape
    if out is None:
        out = torch.empty((M, K // 32 * 36), dtype=torch.uint8, device=x.device)
    if norm_weight.dtype != torch.float16 or norm_weight.numel() != K:
        raise TypeError("norm_weight must be float16 [K]")
    if x.dtype not in (torch.float32, torch.float16):
        raise TypeError("x must be float32 or float16")
    dt = OUT_F16 if x.dtype == torch.float16 else OUT_F32
    rc = _lib.load().ifx_rmsnorm_quantize_q8_1(_dev(x, "x"), dt, _dev(norm_weight, "norm_weight"),
                                               _dev(out, "out"), M, K, float(eps), _stream(stream))
    _check(rc, "ifx_rmsnorm_quantize_q8_1")
    return out


def silu_mul_quantize_q8_1(gate, up, out=None, stream=None):
    """SiLU(gate) * up for fp32/fp16 [M, K], then Q8_1."""
    M, K = gate.shape
    if up.shape != gate.shape or up.dtype != gate.dtype:
        raise ValueError("gate and up must match")
    if gate.dtype not in (torch.float32, torch.float16):
        raise TypeError("gate/up must be float32 or float16")
    if out is None:
        out = torch.empty((M, K // 32 * 36), dtype=torch.uint8, device=gate.device)
    dt = OUT_F16 if gate.dtype == torch.float16 else OUT_F32
    rc = _lib.load().ifx_silu_mul_quantize_q8_1(_dev(gate, "gate"), _dev(up, "up"), dt,
                                                _dev(out, "out"), M, K, _stream(stream))
    _check(rc, "ifx_silu_mul_quantize_q8_1")
    return out


IN_BF16 = 2  # the row-symmetric quantizers also take bf16 input


def _rows_dtype(t):
    return {torch.float32: OUT_F32, torch.float16: OUT_F16, torch.bfloat16: IN_BF16}[t.dtype]


def quantize_rows_symmetric(x, codes=None, scales=None, stream=None):
    """Per-row symmetric int8 codes and fp32 row scales of x [M, K]
    (fp32 / fp16 / bf16): the packed-activation format of qgemv_packed."""
    M, K = x.shape
    if codes is None:
        codes = torch.empty((M, K), dtype=torch.int8, device=x.device)
    if scales is None:
        scales = torch.empty(M, dtype=torch.float32, device=x.device)
    rc = _lib.load().ifx_quantize_rows_symmetric(_dev(x, "x"), _rows_dtype(x), _dev(codes, "codes"),
                                                 _dev(scales, "scales"), M, K, _stream(stream))
    _check(rc, "ifx_quantize_rows_symmetric")
    return codes, scales


def silu_mul_quantize_rows_symmetric(gate, up, codes=None, scales=None, stream=None):
    """quantize_rows_symmetric of SiLU(gate) * up."""
    M, K = gate.shape
    if up.shape != gate.shape or up.dtype != gate.dtype:
        raise ValueError("gate and up must match")
    if codes is None:
        codes = torch.empty((M, K), dtype=torch.int8, device=gate.device)
    if scales is None:
        scales = torch.empty(M, dtype=torch.float32, device=gate.device)
    rc = _lib.load().ifx_silu_mul_quantize_rows_symmetric(
        _dev(gate, "gate"), _dev(up, "up"), _rows_dtype(gate), _dev(codes, "codes"),
        _dev(scales, "scales"), M, K, _stream(stream))
    _check(rc, "ifx_silu_mul_quantize_rows_symmetric")
    return codes, scales


def qgemv_packed(qtype, Ws, codes, scales, M, Ns, K, outs=None, stream=None):
    """fp16 [M, N_i] = row_scale * (W_i . codes) for 1..3 projections of raw
    GGUF weights over packed (per-row symmetric int8) activations."""
    import ctypes
    count = len(Ws)
    if not 1 <= count <= 3 or len(Ns) != count:
        raise ValueError("1..3 projections with one N each")
    if outs is None:
        outs = [torch.empty((M, n), dtype=torch.float16, device=codes.device) for n in Ns]
    for W, n, out in zip(Ws, Ns, outs):
        if W.numel() < weight_bytes(qtype, n, K):
            raise ValueError("W is smaller than N x K blocks")
        if out.numel() < M * n or out.dtype != torch.float16:
            raise ValueError("bad output tensor")
    if codes.numel() < M * K or codes.dtype != torch.int8 or scales.numel() < M:
        raise ValueError("codes / scales smaller than M x K / M")
    wp = (ctypes.c_void_p * count)(*[_dev(w, "W") for w in Ws])
    yp = (ctypes.c_void_p * count)(*[_dev(y, "out") for y in outs])
    nn = (ctypes.c_int * count)(*Ns)
    rc = _lib.load().ifx_qgemv_packed(qtype, count, wp, yp, nn, _dev(codes, "codes"),
                                      _dev(scales, "scales"), M, K, _stream(stream))
    _check(rc, "ifx_qgemv_packed")
    return outs


def qgemv(qtype, W, A, M, N, K, out=None, out_dtype=torch.float32, mode=STORE, bias=None,
          stream=None, prefill=False, workspace=None):
    """y [M, N] (op)= W . a with raw GGUF W and Q8_1 A (all device tensors).
    workspace: a uint8 device tensor (qgemv_workspace_bytes, zeroed once)
    for the deterministic K-split reduction (ifx_qgemv_ws)."""
    if out is None:
        out = torch.empty((M, N), dtype=out_dtype, device=W.device)
    od = OUT_F16 if out.dtype == torch.float16 else OUT_F32
    if out.dtype not in (torch.float16, torch.float32):
        raise TypeError("out must be float32 or float16")
    if (qtype in BLOCK_BYTES or qtype in (Q8_0_R, Q6_K_R, Q8_0_T, Q4_K_T, Q6_K_T)) and \
            W.numel() < weight_bytes(qtype, N, K):
        raise ValueError("W is smaller than N x K blocks")
    if A.numel() < M * (K // 32) * 36:
        raise ValueError("A is smaller than M x K/32 Q8_1 blocks")
    if out.numel() < M * N:
        raise ValueError("out is smaller than M x N")
    bptr = _dev(bias, "bias") if bias is not None else None
    if workspace is not None:
        rc = _lib.load().ifx_qgemv_ws(qtype, _dev(W, "W"), _dev(A, "A"), _dev(out, "out"), od,
                                      mode, bptr, M, N, K, _dev(workspace, "workspace"),
                                      workspace.numel() * workspace.element_size(),
                                      _stream(stream))
        _check(rc, "ifx_qgemv_ws")
        return out
    fn = _lib.load().ifx_qgemm_prefill if prefill else _lib.load().ifx_qgemv
    rc = fn(qtype, _dev(W, "W"), _dev(A, "A"), _dev(out, "out"), od, mode, bptr, M, N, K,
            _stream(stream))
    _check(rc, "ifx_qgemm_prefill" if prefill else "ifx_qgemv")
    return out


def qgemv_workspace_bytes(qtype, Ns, M, K, out_dtype=torch.float32):
    """Bytes of workspace the deterministic split of qgemv / qgemv_grouped
    needs for projections of Ns rows (0: the launch does not split)."""
    import ctypes
    nn = (ctypes.c_int * len(Ns))(*Ns)
    od = OUT_F16 if out_dtype == torch.float16 else OUT_F32
    return int(_lib.load().ifx_qgemv_workspace_bytes(qtype, len(Ns), nn, od, M, K))


def prefill_workspace_bytes(qtype, M, N, K):
    """Bytes of workspace qgemm_prefill_ws uses at this shape (0: none)."""
    return int(_lib.load().ifx_qgemm_prefill_workspace_bytes(qtype, M, N, K))


def qgemm_prefill_ws(qtype, W, A, M, N, K, workspace, out=None, out_dtype=torch.float32,
                     mode=STORE, bias=None, stream=None):
    """The prefill GEMM with a caller-owned workspace (a device tensor of at
    least prefill_workspace_bytes bytes): the fp16 activations are converted
    once into it; bit-identical to qgemv(..., prefill=True)."""
    if out is None:
        out = torch.empty((M, N), dtype=out_dtype, device=W.device)
    od = OUT_F16 if out.dtype == torch.float16 else OUT_F32
    if W.numel() < weight_bytes(qtype, N, K) or A.numel() < M * (K // 32) * 36 or out.numel() < M * N:
        raise ValueError("W, A or out is smaller than the shape")
    nbytes = workspace.numel() * workspace.element_size()
    bptr = _dev(bias, "bias") if bias is not None else None
    rc = _lib.load().ifx_qgemm_prefill_ws(qtype, _dev(W, "W"), _dev(A, "A"), _dev(out, "out"), od,
                                          mode, bptr, M, N, K, _dev(workspace, "workspace"), nbytes,
                                          _stream(stream))
    _check(rc, "ifx_qgemm_prefill_ws")
    return out


def prefill_ordered_workspace_bytes(qtype, M, N, K, out_dtype=torch.float32):
    """Bytes of workspace qgemm_prefill_ordered needs at this shape."""
    od = OUT_F16 if out_dtype == torch.float16 else OUT_F32
    return int(_lib.load().ifx_qgemm_prefill_ordered_workspace_bytes(qtype, od, M, N, K))


def qgemm_prefill_ordered(qtype, W, A, M, N, K, workspace, out=None, out_dtype=torch.float32,
                          mode=STORE, bias=None, stream=None):
    """The prefill GEMM with its K split reduced in split order through the
    workspace (a device tensor of at least prefill_ordered_workspace_bytes
    bytes, 256-byte aligned): the same bits on every call."""
    if out is None:
        out = torch.empty((M, N), dtype=out_dtype, device=W.device)
    od = OUT_F16 if out.dtype == torch.float16 else OUT_F32
    if W.numel() < weight_bytes(qtype, N, K) or A.numel() < M * (K // 32) * 36 or out.numel() < M * N:
        raise ValueError("W, A or out is smaller than the shape")
    nbytes = workspace.numel() * workspace.element_size()
    bptr = _dev(bias, "bias") if bias is not None else None
    rc = _lib.load().ifx_qgemm_prefill_ordered(qtype, _dev(W, "W"), _dev(A, "A"), _dev(out, "out"),
                                               od, mode, bptr, M, N, K,
                                               _dev(workspace, "workspace"), nbytes,
                                               _stream(stream))
    _check(rc, "ifx_qgemm_prefill_ordered")
    return out


def qgemm_prefill_noalloc(qtype, W, A, M, N, K, out=None, out_dtype=torch.float32, mode=STORE,
                          bias=None, stream=None):
    """qgemm_prefill_ws with the library's static device scratch as the
    workspace (ifx_qgemm_prefill_noalloc): the call allocates nothing (pass
    `out` to keep this wrapper from allocating too).  Calls that overlap on
    one GPU race on the scratch."""
    if out is None:
        out = torch.empty((M, N), dtype=out_dtype, device=W.device)
    od = OUT_F16 if out.dtype == torch.float16 else OUT_F32
    if W.numel() < weight_bytes(qtype, N, K) or A.numel() < M * (K // 32) * 36 or out.numel() < M * N:
        raise ValueError("W, A or out is smaller than the shape")
    bptr = _dev(bias, "bias") if bias is not None else None
    rc = _lib.load().ifx_qgemm_prefill_noalloc(qtype, _dev(W, "W"), _dev(A, "A"), _dev(out, "out"),
                                               od, mode, bptr, M, N, K, _stream(stream))
    _check(rc, "ifx_qgemm_prefill_noalloc")
    return out


NOALLOC_SCRATCH_BYTES = 16 << 20  # IFX_NOALLOC_SCRATCH_BYTES


PREFILL_INT8, PREFILL_F16, DECODE_DQ_F16 = 1, 2, 3


def qgemm_prefill_kernel(qtype, W, A, M, N, K, kernel, splits=0, out=None,
                         out_dtype=torch.float32, mode=STORE, bias=None, stream=None):
    """The prefill GEMM on an explicit kernel (PREFILL_INT8: integer-exact
    int8 MFMA; PREFILL_F16: in-kernel dequant to fp16 + fp16 MFMA).  splits
    forces the K split of the fp16 kernel (0 = chosen from the shape)."""
    if out is None:
        out = torch.empty((M, N), dtype=out_dtype, device=W.device)
    od = OUT_F16 if out.dtype == torch.float16 else OUT_F32
    if W.numel() < weight_bytes(qtype, N, K) or A.numel() < M * (K // 32) * 36 \
            or out.numel() < M * N:
        raise ValueError("W, A or out is smaller than the shape")
    bptr = _dev(bias, "bias") if bias is not None else None
    rc = _lib.load().ifx_qgemm_prefill_kernel(qtype, _dev(W, "W"), _dev(A, "A"),
                                              _dev(out, "out"), od, mode, bptr, M, N, K,
                                              kernel, splits, _stream(stream))
    _check(rc, "ifx_qgemm_prefill_kernel")
    return out


def qgemv_grouped(qtype, Ws, A, M, Ns, K, outs=None, out_dtype=torch.float32, mode=STORE,
                  stream=None, workspace=None):
    """Sibling projections over one Q8_1 A: [W_i . a for W_i in Ws], one launch
    for M <= 2.  Returns the list of outputs [M, N_i]."""
    import ctypes
    count = len(Ws)
    if not 1 <= count <= 3 or len(Ns) != count:
        raise ValueError("1..3 projections with one N each")
    if outs is None:
        outs = [torch.empty((M, n), dtype=out_dtype, device=A.device) for n in Ns]
    for W, n, out in zip(Ws, Ns, outs):
        if W.numel() < weight_bytes(qtype, n, K):
            raise ValueError("W is smaller than N x K blocks")
        if out.numel() < M * n or out.dtype != outs[0].dtype:
            raise ValueError("bad output tensor")
    if A.numel() < M * (K // 32) * 36:
        raise ValueError("A is smaller than M x K/32 Q8_1 blocks")
    od = OUT_F16 if outs[0].dtype == torch.float16 else OUT_F32
    wp = (ctypes.c_void_p * count)(*[_dev(w, "W") for w in Ws])
    yp = (ctypes.c_void_p * count)(*[_dev(y, "out") for y in outs])
    nn = (ctypes.c_int * count)(*Ns)
    if workspace is not None:
        rc = _lib.load().ifx_qgemv_grouped_ws(qtype, count, wp, yp, nn, _dev(A, "A"), od, mode, M,
                                              K, _dev(workspace, "workspace"),
                                              workspace.numel() * workspace.element_size(),
                                              _stream(stream))
        _check(rc, "ifx_qgemv_grouped_ws")
        return outs
    rc = _lib.load().ifx_qgemv_grouped(qtype, count, wp, yp, nn, _dev(A, "A"), od, mode, M, K,
                                       _stream(stream))
    _check(rc, "ifx_qgemv_grouped")
    return outs


def qgemv_grouped_rmsnorm(qtype, Ws, x, norm_weight, M, Ns, K, eps=1e-6, outs=None,
                          out_dtype=torch.float32, mode=STORE, stream=None):
    """RMSNorm + Q8_1 of the residual x [M, K] (fp32/fp16) fused into the
    grouped GEMV over Ws (Q4_K, M <= 2); norm_weight None: the plain Q8_1
    quantizer instead.  Returns the list of outputs."""
    import ctypes
    count = len(Ws)
    if outs is None:
        outs = [torch.empty((M, N), dtype=out_dtype, device=Ws[0].device) for N in Ns]
    od = OUT_F16 if outs[0].dtype == torch.float16 else OUT_F32
    xd = OUT_F16 if x.dtype == torch.float16 else OUT_F32
    if x.numel() < M * K or (norm_weight is not None and norm_weight.numel() < K):
        raise ValueError("x or norm_weight is smaller than the shape")
    for W, N, Y in zip(Ws, Ns, outs):
        if W.numel() < weight_bytes(qtype, N, K) or Y.numel() < M * N:
            raise ValueError("W or out is smaller than the shape")
    wp = (ctypes.c_void_p * count)(*[_dev(w, "W") for w in Ws])
    yp = (ctypes.c_void_p * count)(*[_dev(y, "out") for y in outs])
    npp = (ctypes.c_int * count)(*Ns)
    nwp = _dev(norm_weight, "norm_weight") if norm_weight is not None else None
    rc = _lib.load().ifx_qgemv_grouped_rmsnorm(qtype, count, wp, yp, npp, _dev(x, "x"), xd,
                                               nwp, eps, od, mode, M, K, _stream(stream))
    _check(rc, "ifx_qgemv_grouped_rmsnorm")
    return outs


def gate_up_silu_workspace_bytes(qtype, M, N, K):
    """Workspace bytes qgemv_gate_up_silu needs (0: none)."""
    return int(_lib.load().ifx_qgemv_gate_up_silu_workspace_bytes(qtype, M, N, K))


def qgemv_gate_up_silu(qtype, Wg, Wu, A, M, N, K, h_out=None, q8_1_out=None, want_h=True,
                       want_q8_1=True, h_dtype=torch.float32, stream=None, workspace=None):
    """h = silu(Wg . a) * (Wu . a) in one launch; returns (h [M, N] or
    None, Q8_1 [M, N/32*36] or None).  workspace: a zeroed uint8 device
    tensor of gate_up_silu_workspace_bytes (the fp16-dequant GEMV's K split
    at M up to 32)."""
    if want_h and h_out is None:
        h_out = torch.empty((M, N), dtype=h_dtype, device=A.device)
    if want_q8_1 and q8_1_out is None:
        q8_1_out = torch.empty((M, N // 32 * 36), dtype=torch.uint8, device=A.device)
    for W in (Wg, Wu):
        if W.numel() < weight_bytes(qtype, N, K):
            raise ValueError("W is smaller than N x K blocks")
    if h_out is not None and (h_out.numel() < M * N or
                              h_out.dtype not in (torch.float32, torch.float16)):
        raise ValueError("bad h output")
    if q8_1_out is not None and q8_1_out.numel() < M * (N // 32) * 36:
        raise ValueError("bad Q8_1 output")
    hd = OUT_F16 if h_out is not None and h_out.dtype == torch.float16 else OUT_F32
    hp = _dev(h_out, "h") if h_out is not None else None
    qp = _dev(q8_1_out, "q8_1_out") if q8_1_out is not None else None
    if workspace is not None:
        rc = _lib.load().ifx_qgemv_gate_up_silu_ws(
            qtype, _dev(Wg, "Wg"), _dev(Wu, "Wu"), _dev(A, "A"), hp, hd, qp, M, N, K,
            _dev(workspace, "workspace"), workspace.numel() * workspace.element_size(),
            _stream(stream))
        _check(rc, "ifx_qgemv_gate_up_silu_ws")
        return h_out, q8_1_out
    rc = _lib.load().ifx_qgemv_gate_up_silu(qtype, _dev(Wg, "Wg"), _dev(Wu, "Wu"), _dev(A, "A"),
                                            hp, hd, qp, M, N, K, _stream(stream))
    _check(rc, "ifx_qgemv_gate_up_silu")
    return h_out, q8_1_out


def qgemv_gate_up_silu_rmsnorm(qtype, Wg, Wu, x, norm_weight, M, N, K, eps=1e-6, h_out=None,
                               q8_1_out=None, want_h=True, want_q8_1=True,
                               h_dtype=torch.float32, stream=None):
    """qgemv_gate_up_silu with the RMSNorm + Q8_1 producer of the residual
    x [M, K] (fp32/fp16) fused in (Q4_K, M <= 2, K <= 2048); returns
    (h or None, Q8_1 or None)."""
    if want_h and h_out is None:
        h_out = torch.empty((M, N), dtype=h_dtype, device=x.device)
    if want_q8_1 and q8_1_out is None:
        q8_1_out = torch.empty((M, N // 32 * 36), dtype=torch.uint8, device=x.device)
    for W in (Wg, Wu):
        if W.numel() < weight_bytes(qtype, N, K):
            raise ValueError("W is smaller than N x K blocks")
    if x.numel() < M * K or norm_weight.numel() < K:
        raise ValueError("x or norm_weight is smaller than the shape")
    if h_out is not None and (h_out.numel() < M * N or
                              h_out.dtype not in (torch.float32, torch.float16)):
        raise ValueError("bad h output")
    if q8_1_out is not None and q8_1_out.numel() < M * (N // 32) * 36:
        raise ValueError("bad Q8_1 output")
    hd = OUT_F16 if h_out is not None and h_out.dtype == torch.float16 else OUT_F32
    xd = OUT_F16 if x.dtype == torch.float16 else OUT_F32
    rc = _lib.load().ifx_qgemv_gate_up_silu_rmsnorm(
        qtype, _dev(Wg, "Wg"), _dev(Wu, "Wu"), _dev(x, "x"), xd, _dev(norm_weight, "norm_weight"),
        eps, _dev(h_out, "h") if h_out is not None else None, hd,
        _dev(q8_1_out, "q8_1_out") if q8_1_out is not None else None, M, N, K, _stream(stream))
    _check(rc, "ifx_qgemv_gate_up_silu_rmsnorm")
    return h_out, q8_1_out


def _row_split_bytes(qtype, K):
    n = K + K // 32 * 2 if qtype == Q8_0_R else K // 2 + K // 4 + K // 16 + K // 256 * 2
    return (n + 15) // 16 * 16


def repack(qtype, W, n_rows, K, out=None, stream=None):
    """Row-split copy of raw Q8_0 / Q6_K rows (ifx_repack); returns
    (repacked type, device tensor).  For the M <= 2 GEMV."""
    rt = {Q8_0: Q8_0_R, Q6_K: Q6_K_R}[qtype]
    nbytes = int(_lib.load().ifx_repacked_bytes(qtype, n_rows, K))
    if out is None:
        out = torch.empty(nbytes, dtype=torch.uint8, device=W.device)
    if W.numel() < weight_bytes(qtype, n_rows, K) or out.numel() < nbytes:
        raise ValueError("W or out is smaller than the shape")
    rc = _lib.load().ifx_repack(qtype, _dev(W, "W"), _dev(out, "out"), n_rows, K, _stream(stream))
    _check(rc, "ifx_repack")
    return rt, out


def repack_tiled(qtype, W, n_rows, K, out=None, stream=None):
    """Tiled copy of raw Q4_K / Q6_K / Q8_0 rows (ifx_repack_tiled): returns
    (tiled type, device tensor).  For the MFMA batch GEMVs, M <= 32."""
    tt = {Q4_K: Q4_K_T, Q6_K: Q6_K_T, Q8_0: Q8_0_T}[qtype]
    nbytes = int(_lib.load().ifx_tiled_bytes(qtype, n_rows, K))
    if out is None:
        out = torch.empty(nbytes, dtype=torch.uint8, device=W.device)
    if W.numel() < weight_bytes(qtype, n_rows, K) or out.numel() < nbytes:
        raise ValueError("W or out too small")
    rc = _lib.load().ifx_repack_tiled(qtype, _dev(W, "W"), _dev(out, "out"), n_rows, K,
                                      _stream(stream))
    _check(rc, "ifx_repack_tiled")
    return tt, out


def mmq_layout(qtype, W, n_rows, K, out=None, stream=None):
    """Down-projection MMQ layout of raw Q4_K / Q6_K / Q8_0 rows
    (ifx_mmq_layout_build): the tiled copy plus a row-major copy for M <= 2,
    in one 256-byte-aligned uint8 device tensor."""
    nbytes = int(_lib.load().ifx_mmq_layout_bytes(qtype, n_rows, K))
    if nbytes == 0:
        raise ValueError("no MMQ layout for this type / K")
    if out is None:
        out = torch.empty(nbytes, dtype=torch.uint8, device=W.device)
    if W.numel() < weight_bytes(qtype, n_rows, K) or out.numel() < nbytes:
        raise ValueError("W or out too small")
    rc = _lib.load().ifx_mmq_layout_build(qtype, _dev(W, "W"), _dev(out, "out"), n_rows, K,
                                          _stream(stream))
    _check(rc, "ifx_mmq_layout_build")
    return out


def qgemv_mmq(qtype, layout, A, M, N, K, out=None, out_dtype=torch.float32, mode=STORE,
              ordered=False, stream=None):
    """y [M, N] (op)= W . a on an MMQ layout (ifx_qgemv_mmq), 1 <= M <= 32;
    ordered: K splits added in split order through the layout's workspace."""
    if out is None:
        out = torch.empty((M, N), dtype=out_dtype, device=layout.device)
    od = OUT_F16 if out.dtype == torch.float16 else OUT_F32
    if out.dtype not in (torch.float16, torch.float32):
        raise TypeError("out must be float32 or float16")
    if layout.numel() < int(_lib.load().ifx_mmq_layout_bytes(qtype, N, K)):
        raise ValueError("layout is smaller than N x K")
    if A.numel() < M * (K // 32) * 36 or out.numel() < M * N:
        raise ValueError("A or out too small")
    rc = _lib.load().ifx_qgemv_mmq(qtype, _dev(layout, "layout"), _dev(A, "A"), _dev(out, "out"),
                                   od, mode, M, N, K, int(bool(ordered)), _stream(stream))
    _check(rc, "ifx_qgemv_mmq")
    return out


def dequantize(qtype, W, n_rows, K, out_dtype=torch.float32, stream=None, out=None):
    if out is None:
        out = torch.empty((n_rows, K), dtype=out_dtype, device=W.device)
    od = OUT_F16 if out.dtype == torch.float16 else OUT_F32
    if W.numel() < weight_bytes(qtype, n_rows, K) or out.numel() < n_rows * K:
        raise ValueError("W or out is smaller than n_rows x K")
    rc = _lib.load().ifx_dequantize(qtype, _dev(W, "W"), _dev(out, "out"), od, n_rows, K,
                                    _stream(stream))
    _check(rc, "ifx_dequantize")
    return out


def supports(qtype, M, N, K):
    return bool(_lib.load().ifx_supports(qtype, M, N, K))


def kernel_family(qtype, M, N, K):
    """Kernel family ifx_qgemv runs the shape on (include/ifx_qgemm.h)."""
    return int(_lib.load().ifx_kernel_family(qtype, M, N, K))


class launch_log:
    """Records the kernel instances the entry points called inside the
    `with` block launch on this thread (ifx_launch_log_begin/_end,
    include/ifx_qgemm.h).  dry=True launches nothing: no HIP call is made, so
    the dispatch of any shape can be read on a host without a GPU (use fake
    non-null pointers then).  After the block, `.kernels` is the list of
    instance names, e.g. ["k_gemv<12,1,2,1,4,0,2>"]."""

    def __init__(self, dry=False):
        self.dry = dry
        self.kernels = []

    def __enter__(self):
        _lib.load().ifx_launch_log_begin(1 if self.dry else 0)
        return self

    def __exit__(self, *exc):
        text = _lib.load().ifx_launch_log_end().decode()
        self.kernels = text.split(";") if text else []
        return False
