"""CPU checks of the C ABI: the library loads, exports every entry point
include/ifx_qgemm.h and include/ifx_gguf.h declare, and its host-side validation answers without
touching a GPU (the reference's `false` = a positive status)."""
import ctypes
import os
import re
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADERS = [os.path.join(ROOT, "include", h) for h in ("ifx_qgemm.h", "ifx_gguf.h")]


def declared_symbols():
    text = "".join(open(h).read() for h in HEADERS)
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\s*\*?\s*(ifx_\w+)\s*\(", text, re.M)))


@pytest.fixture(scope="module")
def lib():
    from inferflux_amd import _lib
    return _lib.load()


def test_header_declares_expected_entry_points():
    syms = declared_symbols()
    for s in ("ifx_q8_1_quantize_f32", "ifx_q8_1_quantize_f16", "ifx_qgemv",
              "ifx_qgemm_prefill", "ifx_dequantize", "ifx_supports", "ifx_gguf_open",
              "ifx_gguf_upload", "ifx_gguf_tensor_bytes"):
        assert s in syms


def test_library_exports_every_declared_symbol(lib):
    from inferflux_amd import _lib
    syms = declared_symbols()
    for s in syms:
        assert hasattr(lib, s), s
        assert s in _lib.SIGNATURES, f"{s} has no ctypes signature"
    out = subprocess.run(["nm", "-D", "--defined-only", _lib.LIB_PATH], capture_output=True,
                         text=True, check=True).stdout
    exported = set(re.findall(r"\bT (ifx_\w+)", out))
    assert set(syms) <= exported


def test_library_has_gfx950_code_object():
    """The fat binary embedded in our own build names its offload target."""
    from inferflux_amd import _lib
    data = open(_lib.LIB_PATH, "rb").read()
    assert b"gfx950" in data


def test_block_geometry(lib):
    assert (lib.ifx_block_bytes(12), lib.ifx_block_elems(12)) == (144, 256)
    assert (lib.ifx_block_bytes(14), lib.ifx_block_elems(14)) == (210, 256)
    assert (lib.ifx_block_bytes(8), lib.ifx_block_elems(8)) == (34, 32)
    assert (lib.ifx_block_bytes(9), lib.ifx_block_elems(9)) == (36, 32)
    assert (lib.ifx_block_bytes(13), lib.ifx_block_elems(13)) == (176, 256)
    assert (lib.ifx_block_bytes(15), lib.ifx_block_elems(15)) == (292, 256)
    assert lib.ifx_block_bytes(0) == 0 and lib.ifx_block_elems(16) == 0


def test_supports(lib):
    assert lib.ifx_supports(12, 1, 11008, 2048) == 1
    assert lib.ifx_supports(12, 512, 27648, 5120) == 1
    assert lib.ifx_supports(14, 32, 5120, 13824) == 1
    assert lib.ifx_supports(8, 8, 151936, 2048) == 1
    assert lib.ifx_supports(8, 1, 16, 96) == 1        # Q8_0 needs K % 32 only
    assert lib.ifx_supports(12, 1, 16, 96) == 0       # K-quants need K % 256
    assert lib.ifx_supports(13, 1, 16, 256) == 1      # Q5_K: GEMV, M <= 64
    assert lib.ifx_supports(15, 64, 16, 256) == 1     # Q8_K: GEMV, M <= 64
    assert lib.ifx_supports(15, 65, 16, 256) == 0     # the reference's limit
    assert lib.ifx_supports(13, 1, 16, 128) == 0
    assert lib.ifx_supports(11, 1, 16, 256) == 0      # Q3_K: no kernel
    assert lib.ifx_supports(12, 0, 16, 256) == 0
    # W and A stay below 0xF0000000 bytes, the offset at which the kernels'
    # loads that must read zeros are placed; K up to 2^24
    assert lib.ifx_supports(8, 16, 151936, 24832) == 1  # Q8_0 W 4.009e9 B
    assert lib.ifx_supports(8, 16, 151936, 24960) == 0  # 4.029e9 B >= 0xF0000000
    assert lib.ifx_supports(12, 1, 1, 1 << 24) == 1
    assert lib.ifx_supports(12, 1, 1, (1 << 24) + 256) == 0
    assert lib.ifx_supports(12, 213, 1, 1 << 24) == 1    # A 4.020e9 B
    assert lib.ifx_supports(12, 214, 1, 1 << 24) == 0    # A 4.039e9 B


def test_validation_without_launch(lib):
    """Rejected calls return before any HIP call, so they run on the CPU."""
    fake = ctypes.c_void_p(0x1000)
    # NULL pointers
    assert lib.ifx_qgemv(12, None, fake, fake, 0, 0, None, 1, 16, 256, None) == 3
    assert lib.ifx_qgemv(12, fake, None, fake, 0, 0, None, 1, 16, 256, None) == 3
    assert lib.ifx_qgemv(12, fake, fake, fake, 0, 2, None, 1, 16, 256, None) == 3  # bias mode
    assert lib.ifx_q8_1_quantize_f32(None, fake, 1, 32, None) == 3
    # unsupported type / geometry / mode / dtype
    assert lib.ifx_qgemv(11, fake, fake, fake, 0, 0, None, 1, 16, 256, None) == 1
    assert lib.ifx_qgemv(15, fake, fake, fake, 0, 0, None, 65, 16, 256, None) == 2  # Q8_K, M > 64
    assert lib.ifx_qgemm_prefill(13, fake, fake, fake, 0, 0, None, 8, 16, 256, None) == 1
    assert lib.ifx_qgemv(12, fake, fake, fake, 0, 0, None, 1, 16, 250, None) == 2
    assert lib.ifx_qgemv(12, fake, fake, fake, 0, 0, None, 0, 16, 256, None) == 2
    assert lib.ifx_qgemv(12, fake, fake, fake, 0, 7, None, 1, 16, 256, None) == 2
    assert lib.ifx_qgemv(12, fake, fake, fake, 5, 0, None, 1, 16, 256, None) == 2
    assert lib.ifx_qgemm_prefill(6, fake, fake, fake, 0, 0, None, 64, 16, 256, None) == 1
    assert lib.ifx_q8_1_quantize_f32(fake, fake, 1, 33, None) == 2
    assert lib.ifx_dequantize(12, fake, fake, 0, 4, 100, None) == 2
    assert lib.ifx_status_string(3) == b"null pointer"


def test_packed_validation_without_launch(lib):
    """The packed-activation entries reject bad calls before any HIP call:
    types outside Q4_K / Q6_K / Q8_0 / Q8_K, K off the block size, 0 or 4
    projections, NULL pointers, unknown input dtypes."""
    fake = ctypes.c_void_p(0x1000)
    W = (ctypes.c_void_p * 3)(fake, fake, fake)
    Y = (ctypes.c_void_p * 3)(fake, fake, fake)
    N = (ctypes.c_int * 3)(16, 16, 16)
    packed = lib.ifx_qgemv_packed
    assert packed(13, 1, W, Y, N, fake, fake, 1, 256, None) == 1  # Q5_K: no packed kernel
    assert packed(9, 1, W, Y, N, fake, fake, 1, 256, None) == 1
    assert packed(12, 1, W, Y, N, fake, fake, 1, 250, None) == 2
    assert packed(8, 1, W, Y, N, fake, fake, 1, 48, None) == 2
    assert packed(12, 0, W, Y, N, fake, fake, 1, 256, None) == 2
    assert packed(12, 4, W, Y, N, fake, fake, 1, 256, None) == 2
    assert packed(12, 1, W, Y, N, None, fake, 1, 256, None) == 3
    assert packed(12, 1, W, Y, N, fake, None, 1, 256, None) == 3
    Wn = (ctypes.c_void_p * 3)(fake, None, fake)
    assert packed(12, 2, Wn, Y, N, fake, fake, 1, 256, None) == 3
    Nz = (ctypes.c_int * 3)(16, 0, 16)
    assert packed(12, 2, W, Y, Nz, fake, fake, 1, 256, None) == 2
    assert packed(12, 1, W, Y, N, fake, fake, -1, 256, None) == 2
    assert lib.ifx_quantize_rows_symmetric(None, 0, fake, fake, 1, 8, None) == 3
    assert lib.ifx_quantize_rows_symmetric(fake, 3, fake, fake, 1, 8, None) == 2
    assert lib.ifx_quantize_rows_symmetric(fake, 0, fake, fake, 1, 0, None) == 2
    assert lib.ifx_silu_mul_quantize_rows_symmetric(fake, None, 1, fake, fake, 1, 8, None) == 3


def test_product_fails_loudly_without_library(monkeypatch):
    from inferflux_amd import _lib
    monkeypatch.setattr(_lib, "_lib", None)
    monkeypatch.setattr(_lib, "LIB_PATH", "/nonexistent/libifx_qgemm.so")
    with pytest.raises(_lib.IfxError):
        _lib.load()


def test_product_never_imports_oracle():
    pkg = os.path.join(ROOT, "inferflux_amd")
    for dirpath, _, files in os.walk(pkg):
        for f in files:
            if f.endswith((".py", ".hip", ".h", ".cpp")):
                text = open(os.path.join(dirpath, f)).read()
                assert "oracle" not in re.sub(r"(#|//).*", "", text), f
