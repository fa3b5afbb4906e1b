"""Dispatch routing on the CPU: every launch the benchmark times goes to the
kernel instance tests/launch_table.py names.  The C ABI runs in dry-run mode
(ifx_launch_log_begin(1)): it validates, picks and records the kernel, and
makes no HIP call, so fake non-null pointers stand in for device memory."""
import ctypes

import pytest

from tests.launch_table import IDS, LAUNCHES

_P = ctypes.c_void_p


def _fake(i):
    return _P(0x100000 * (i + 1))


def dry_dispatch(entry, qt, M, Ns, K):
    """Calls the entry point of `entry` in dry-run mode; returns (status,
    kernel instance names)."""
    from inferflux_amd import _lib, ops
    L = _lib.load()
    n = len(Ns)
    W = (_P * n)(*[_fake(i) for i in range(n)])
    Y = (_P * n)(*[_fake(4 + i) for i in range(n)])
    NN = (ctypes.c_int * n)(*Ns)
    A, X, NW, B = _fake(8), _fake(9), _fake(10), _fake(11)
    WS = _fake(12)  # a workspace "large enough" (1 GB) for the _ws entries
    with ops.launch_log(dry=True) as lg:
        if entry in ("gemv_ws", "gemv_accum_ws"):
            rc = L.ifx_qgemv_ws(qt, W[0], A, Y[0], ops.OUT_F32,
                                ops.ACCUM if entry == "gemv_accum_ws" else ops.STORE, None, M,
                                Ns[0], K, WS, 1 << 30, None)
        elif entry in ("mmq_accum", "mmq_accum_ws"):
            rc = L.ifx_qgemv_mmq(qt, W[0], A, Y[0], ops.OUT_F32, ops.ACCUM, M, Ns[0], K,
                                 int(entry == "mmq_accum_ws"), None)
        elif entry == "grouped_ws":
            rc = L.ifx_qgemv_grouped_ws(qt, n, W, Y, NN, A, ops.OUT_F32, ops.STORE, M, K, WS,
                                        1 << 30, None)
        elif entry in ("gemv", "gemv_accum"):
            rc = L.ifx_qgemv(qt, W[0], A, Y[0], ops.OUT_F32,
                             ops.ACCUM if entry == "gemv_accum" else ops.STORE, None, M, Ns[0], K,
                             None)
        elif entry == "grouped":
            rc = L.ifx_qgemv_grouped(qt, n, W, Y, NN, A, ops.OUT_F32, ops.STORE, M, K, None)
        elif entry in ("grouped_rmsnorm", "quantize_accum"):
            norm = NW if entry == "grouped_rmsnorm" else None
            mode = ops.STORE if entry == "grouped_rmsnorm" else ops.ACCUM
            rc = L.ifx_qgemv_grouped_rmsnorm(qt, n, W, Y, NN, X, ops.OUT_F32, norm, 1e-6,
                                             ops.OUT_F32, mode, M, K, None)
        elif entry == "gate_up_silu_rmsnorm":
            rc = L.ifx_qgemv_gate_up_silu_rmsnorm(qt, W[0], _fake(1), X, ops.OUT_F32, NW, 1e-6,
                                                  None, ops.OUT_F32, B, M, Ns[0], K, None)
        elif entry == "gate_up_silu_ws":
            rc = L.ifx_qgemv_gate_up_silu_ws(qt, W[0], _fake(1), A, None, ops.OUT_F32, B, M, Ns[0],
                                             K, WS, 1 << 30, None)
        elif entry == "gate_up_silu":
            rc = L.ifx_qgemv_gate_up_silu(qt, W[0], _fake(1), A, None, ops.OUT_F32, B, M, Ns[0], K,
                                          None)
        elif entry == "packed":
            rc = L.ifx_qgemv_packed(qt, n, W, Y, NN, A, B, M, K, None)
        elif entry == "prefill":
            rc = L.ifx_qgemm_prefill(qt, W[0], A, Y[0], ops.OUT_F32, ops.STORE, None, M, Ns[0], K,
                                     None)
        elif entry == "prefill_int8":
            rc = L.ifx_qgemm_prefill_kernel(qt, W[0], A, Y[0], ops.OUT_F32, ops.STORE, None, M,
                                            Ns[0], K, ops.PREFILL_INT8, 0, None)
        else:
            raise ValueError(entry)
    return rc, lg.kernels


@pytest.mark.parametrize("lid,entry,qt,M,Ns,K,want", LAUNCHES, ids=IDS)
def test_bench_launch_routing(lid, entry, qt, M, Ns, K, want):
    rc, kernels = dry_dispatch(entry, qt, M, Ns, K)
    assert rc == 0
    assert kernels == want


def test_dry_run_launches_nothing_and_log_closes():
    """Validation still runs in dry-run mode (a bad geometry launches and
    records nothing), and a closed log records nothing further."""
    from inferflux_amd import _lib, ops
    L = _lib.load()
    with ops.launch_log(dry=True) as lg:
        rc = L.ifx_qgemv(ops.Q4_K, _fake(0), _fake(1), _fake(2), ops.OUT_F32, ops.STORE, None,
                         1, 64, 300, None)  # K % 256 != 0
    assert rc == 2 and lg.kernels == []  # IFX_BAD_GEOMETRY
    rc, kernels = dry_dispatch("gemv", ops.Q4_K, 1, (64,), 256)
    assert rc == 0 and len(kernels) == 1
    assert L.ifx_launch_log_end().decode() == ""


def test_tiled_routing():
    """Tiled weights: the slot-packed int8 MFMA GEMV for M <= 16 (wide Q4_K
    launches: M <= 8) and the fp16-dequant MFMA GEMV above (its no-split
    form for 192 or more row groups), both with the layout flag; the
    gate/up/SiLU entry on the slot kernel from M = 1; M > 32 not handled."""
    from inferflux_amd import _lib, ops
    L = _lib.load()
    for M in (1, 2, 5, 8):
        rc, k = dry_dispatch("gemv", ops.Q4_K_T, M, (11008,), 2048)
        assert rc == 0 and k == ["k_gemv_slot<12,8,8,0,0,0,1>"]
    rc, k = dry_dispatch("gemv", ops.Q6_K_T, 8, (2048,), 11008)  # few row groups: K split
    assert rc == 0 and k == ["k_fill_zero", "k_gemv_slot<14,8,4,0,1,0,1>"]
    rc, k = dry_dispatch("grouped", ops.Q4_K_T, 16, (5120, 1024, 1024), 5120)
    assert rc == 0 and k == ["k_gemv_slot<12,16,8,0,0,0,1>"]  # short K: 8 waves, no split
    rc, k = dry_dispatch("grouped", ops.Q4_K_T, 32, (5120, 1024, 1024), 5120)
    assert rc == 0 and k[-1] == "k_gemv_dq<12,0,1,1>"
    for M in (1, 4, 8):
        rc, k = dry_dispatch("gate_up_silu", ops.Q4_K_T, M, (11008,), 2048)
        assert rc == 0 and k == ["k_gemv_slot<12,8,4,0,0,1,1>"]
    assert dry_dispatch("gemv", ops.Q4_K_T, 33, (64,), 256)[0] == 2
    assert dry_dispatch("prefill", ops.Q4_K_T, 512, (64,), 256)[0] == 2
    assert L.ifx_kernel_family(ops.Q4_K_T, 8, 64, 256) == 2
    assert L.ifx_kernel_family(ops.Q6_K_T, 9, 64, 256) == 2  # two 16-row slots
    assert L.ifx_kernel_family(ops.Q4_K_T, 16, 16384, 256) == 5  # wide Q4_K from M = 9
    assert L.ifx_kernel_family(ops.Q6_K_T, 17, 64, 256) == 5
    assert L.ifx_kernel_family(ops.Q6_K_T, 33, 64, 256) == 0
    assert L.ifx_tiled_bytes(ops.Q4_K, 33, 512) == 64 * 2 * 144
    assert L.ifx_tiled_bytes(ops.Q8_0, 33, 512) == 64 * 2 * 272
    assert L.ifx_tiled_bytes(ops.Q5_K, 32, 512) == 0
    rc, k = dry_dispatch("gemv", ops.Q8_0_T, 8, (151936,), 2048)
    assert rc == 0 and k == ["k_gemv_slot<8,8,1,0,0,0,1>"]
    rc, k = dry_dispatch("gemv", ops.Q8_0_T, 32, (151936,), 2048)  # >= 192 row groups: no split
    assert rc == 0 and k == ["k_gemv_dqr<8,0,1,0,4,2,8>"]
