"""The C++ FusedQuantGemm mirror (include/ifx_fused_quant_gemm.h): its
host-only policy cases (thresholds, argument rejection, the
INFERFLUX_DISABLE_FUSED_GEMV switch) run here without a GPU; the device
cases run from tests/test_gpu_parity.py."""
import os
import subprocess

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BIN = os.path.join(ROOT, "tests", "cpp", "test_fused_quant_gemm")


def binary():
    """The test binary; built with tests/cpp/Makefile when missing."""
    if not os.path.exists(BIN):
        subprocess.run(["make", "-s", "-C", os.path.join(ROOT, "oracle")], check=True)
        subprocess.run(["make", "-s", "-C", os.path.dirname(BIN)], check=True)
    return BIN


def test_policy_cases():
    r = subprocess.run([binary(), "policy"], capture_output=True, text=True, timeout=60)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "policy: 0 failure(s)" in r.stdout
