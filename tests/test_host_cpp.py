"""The C++ FusedQuantGemm mirror (include/ifx_fused_quant_gemm.h): its
host-only policy cases (thresholds, argument rejection, the
INFERFLUX_DISABLE_FUSED_GEMV switch) run here without a GPU; the device
cases run from tests/test_gpu_parity.py."""
import os
import subprocess

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BIN = os.path.join(ROOT, "tests", "cpp", "test_fused_quant_gemm")


BIN_MMQ = os.path.join(ROOT, "tests", "cpp", "test_down_proj_mmq")


def binary(path=BIN):
    """A test binary; built with tests/cpp/Makefile when missing."""
    if not os.path.exists(path):
        subprocess.run(["make", "-s", "-C", os.path.join(ROOT, "oracle")], check=True)
        subprocess.run(["make", "-s", "-C", os.path.dirname(path)], check=True)
    return path


def test_policy_cases():
    r = subprocess.run([binary(), "policy"], capture_output=True, text=True, timeout=60)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "policy: 0 failure(s)" in r.stdout


def test_down_proj_and_selection_policy_cases():
    """DownProjMmq / BuildDownProjMmqLayout argument rejection and the
    FfnProj / DownProj operator selectors against the reference's own
    expectations (tests/cpp/test_down_proj_mmq.cpp)."""
    r = subprocess.run([binary(BIN_MMQ), "policy"], capture_output=True, text=True, timeout=60)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "policy: 0 failure(s)" in r.stdout
