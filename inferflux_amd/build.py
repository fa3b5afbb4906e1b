"""Builds libifx_qgemm.so in-tree with hipcc for gfx950.

Run as `python -m inferflux_amd.build` or through __graft_entry__.build().
Every source compiles on every call (the build is the "does it build"
check); objects go to inferflux_amd/_build/, the library next to this file.
"""
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OBJ = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libifx_qgemm.so")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

COMMON = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-Wall",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-I" + os.path.join(HERE, "..", "include"),
]
# IFX_TUNING=1 at build time compiles in the IFX_* environment overrides of
# the dispatch and launch geometry (tuning sweeps only; see ifx_common.h).
if os.environ.get("IFX_TUNING") == "1":
    COMMON.append("-DIFX_TUNING")
    if os.environ.get("IFX_STAMPS") == "1":  # wave timelines (IFX_STAMP)
        COMMON.append("-DIFX_STAMPS")
    # a tuning build goes to its own directory, never over the product library
    OBJ = os.environ.get("IFX_BUILD_OUT", os.path.join(HERE, "_build_tuning"))
    LIB = os.path.join(OBJ, "libifx_qgemm.so")
# Bit-exact kernels: no fp contraction anywhere in these translation units.
EXACT = {"quantize.hip", "dequant.hip"}
SOURCES = ["api.hip", "quantize.hip", "dequant.hip", "gemv.hip", "mmq_skinny.hip", "mmvq.hip", "gemm_mfma.hip", "gemv_lds.hip", "gemv_slot.hip", "gemm_f16.hip", "gemv_dq.hip", "packed.hip",
           "../host/fused_quant_gemm.cpp", "../host/native_dispatch.cpp", "../host/gguf.cpp", "../host/gguf_model.cpp"]


def _run(cmd):
    r = subprocess.run(cmd, capture_output=True, text=True)
    msg = "\n".join(l for l in (r.stdout + r.stderr).splitlines()
                    if "packed-fp32-ops" not in l)
    if r.returncode != 0:
        raise RuntimeError("build failed: " + " ".join(cmd) + "\n" + msg)
    if msg.strip():
        print(msg, file=sys.stderr)


def build(verbose=True):
    os.makedirs(OBJ, exist_ok=True)
    objs = []
    procs = []
    for src in SOURCES:
        obj = os.path.join(OBJ, os.path.basename(src).rsplit(".", 1)[0] + ".o")
        flags = COMMON + (["-ffp-contract=off"] if src in EXACT else [])
        path = os.path.normpath(os.path.join(CSRC, src))
        lang = ["-x", "hip"] if src.endswith(".hip") else []
        cmd = [HIPCC] + flags + ["-c"] + lang + [path, "-o", obj]
        procs.append((cmd, subprocess.Popen(cmd, stdout=subprocess.PIPE,
                                            stderr=subprocess.PIPE, text=True)))
        objs.append(obj)
    for cmd, p in procs:
        out, err = p.communicate()
        msg = "\n".join(l for l in (out + err).splitlines() if "packed-fp32-ops" not in l)
        if p.returncode != 0:
            raise RuntimeError("build failed: " + " ".join(cmd) + "\n" + msg)
        if msg.strip() and verbose:
            print(msg, file=sys.stderr)
    tmp = LIB + ".tmp"
    _run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp] + objs)
    os.replace(tmp, LIB)
    if verbose:
        print("built", LIB)
    return LIB


if __name__ == "__main__":
    build()
