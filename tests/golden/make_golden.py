"""Writes the committed golden fixtures of this directory.

No Python reference implementation exists for this path and the ggml CPU
code is absent from the reference snapshot, so the fixtures are computed
here with numpy straight from the reference's formulas (independently of
the C oracle, which the tests then check against them):
  q8_1_kat.json   the input patterns of the reference's Q8_1 known-answer
                  tests (tests/unit/test_native_forward.cpp:7706-7930) with
                  the codes of the kernel formula rint(x * 127/amax)
                  (fused_dequant_gemv.cuh:597-655) and of the test's own
                  formula lrint(x / (amax/127)), d and s as fp16 bits
  gemv_small.npz  seeded Q4_K/Q6_K/Q8_0 blocks, activations, their Q8_1
                  blocks, fp32 dequantized weights (quant_common.cuh:100-188
                  evaluated in numpy float32) and fp64 products
Run: python tests/golden/make_golden.py
"""
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from inferflux_amd import synth  # noqa: E402
from tests import qref  # noqa: E402

Q8_0, Q4_K, Q6_K = 8, 12, 14


def q8_1_numpy(x):
    """Q8_1 blocks from the kernel formula, numpy float32 throughout."""
    x = np.asarray(x, np.float32)
    M, K = x.shape
    xb = x.reshape(M, K // 32, 32)
    amax = np.abs(xb).max(axis=2)
    d = amax / np.float32(127)
    with np.errstate(divide="ignore"):
        inv = np.where(amax > 0, np.float32(127) / amax, np.float32(0)).astype(np.float32)
    q = np.clip(np.rint(xb * inv[..., None]), -128, 127).astype(np.int32)
    s = d * q.sum(axis=2).astype(np.float32)
    out = np.zeros((M, K // 32, 36), np.uint8)
    out[..., 0:2] = d.astype(np.float16).view(np.uint8).reshape(M, K // 32, 2)
    out[..., 2:4] = s.astype(np.float16).view(np.uint8).reshape(M, K // 32, 2)
    out[..., 4:36] = q.astype(np.int8).view(np.uint8)
    return out.reshape(M, -1), q, d


def kat_cases():
    cases = []
    i = np.arange(32, dtype=np.float32)
    gate = (i - 16) / np.float32(8)
    up = 1 + (np.arange(32) % 5).astype(np.float32) * np.float32(0.25)
    gate = gate.astype(np.float16).astype(np.float32)
    up = up.astype(np.float16).astype(np.float32)
    x1 = gate / (1 + np.exp(-gate)) * up
    i2 = np.arange(64, dtype=np.float32)
    g2 = (np.sin(np.float32(0.19) * i2) * 2).astype(np.float16).astype(np.float32)
    u2 = (np.float32(0.75) + ((np.arange(64) * 3) % 11).astype(np.float32) * np.float32(0.17)
          ).astype(np.float16).astype(np.float32)
    x2 = g2 / (1 + np.exp(-g2)) * u2
    r3 = (np.cos(np.float32(0.11) * i2) * np.float32(1.7)).astype(np.float16).astype(np.float32)
    w3 = (np.float32(0.9) + (np.arange(64) % 7).astype(np.float32) * np.float32(0.03)
          ).astype(np.float16).astype(np.float32)
    rms = np.float32(1) / np.sqrt((r3 * r3).sum() / np.float32(64) + np.float32(1e-5))
    x3 = r3 * rms * w3
    for name, x in (("silu_mul_k32", x1), ("silu_mul_k64", x2), ("rmsnorm_k64", x3)):
        x = x.astype(np.float32).reshape(1, -1)
        blocks, q, d = q8_1_numpy(x)
        q_test = np.clip(np.rint(x.reshape(1, -1, 32) / d[..., None]), -128, 127).astype(np.int32)
        K = x.shape[1]
        b = blocks.reshape(-1, 36)
        cases.append({
            "name": name,
            "x": [float(v) for v in x.ravel()],
            "q": [int(v) for v in q.ravel()],
            "q_ref_test_formula": [int(v) for v in q_test.ravel()],
            "d_bits": [int(v) for v in b[:, 0:2].copy().view(np.uint16).ravel()],
            "s_bits": [int(v) for v in b[:, 2:4].copy().view(np.uint16).ravel()],
            "K": K,
        })
    return cases


def dequant_f32(qtype, w, n, K):
    if qtype == Q4_K:
        b = w.reshape(-1, 144)
        d = b[:, 0:2].copy().view(np.float16).astype(np.float32)
        dmin = b[:, 2:4].copy().view(np.float16).astype(np.float32)
        sc, m = qref.unpack_scale_min_k4(b[:, 4:16])
        qs = b[:, 16:144].reshape(-1, 4, 32).astype(np.int64)
        q = np.stack([qs & 0xF, qs >> 4], axis=2).reshape(-1, 8, 32).astype(np.float32)
        return ((d[:, :, None] * sc[:, :, None].astype(np.float32)) * q
                - dmin[:, :, None] * m[:, :, None].astype(np.float32)).reshape(n, K)
    if qtype == Q6_K:
        b = w.reshape(-1, 210)
        ql = b[:, 0:128].reshape(-1, 2, 2, 32).astype(np.int64)
        qh = b[:, 128:192].reshape(-1, 2, 32).astype(np.int64)
        lo = np.stack([ql[:, :, 0] & 0xF, ql[:, :, 1] & 0xF, ql[:, :, 0] >> 4, ql[:, :, 1] >> 4], 2)
        hi = np.stack([(qh >> (2 * s)) & 3 for s in range(4)], 2)
        q = ((lo | (hi << 4)) - 32).astype(np.float32)
        d = b[:, 208:210].copy().view(np.float16).astype(np.float32)
        sc = np.repeat(b[:, 192:208].view(np.int8).astype(np.float32).reshape(-1, 2, 4, 2), 16, 3)
        return ((d[:, :, None, None] * sc) * q).reshape(n, K)
    b = w.reshape(-1, 34)
    d = b[:, 0:2].copy().view(np.float16).astype(np.float32)
    return (d * b[:, 2:34].view(np.int8).astype(np.float32)).reshape(n, K)


def double_rounding_blocks(n=4):
    """Q8_1 blocks whose s = f16(f32(d * sum)) differs from a single rounding
    f16(d * sum): an implementation that fuses the multiply into the fp16
    conversion fails on them."""
    rng = np.random.default_rng(0)
    found = []
    while len(found) < n:
        x = (rng.standard_normal((4096, 32)) * rng.uniform(0.1, 30)).astype(np.float32)
        _, q, d = q8_1_numpy(x.reshape(1, -1))
        s = q.reshape(-1, 32).astype(np.int64).sum(1)
        single = (d.ravel().astype(np.float64) * s).astype(np.float16)
        double = (d.ravel() * s.astype(np.float32)).astype(np.float16)
        idx = np.nonzero(single != double)[0]
        found.extend(x[i] for i in idx[: n - len(found)])
    x = np.stack(found).reshape(1, -1)
    blocks, _, _ = q8_1_numpy(x)
    return x, blocks


def main():
    with open(os.path.join(HERE, "q8_1_kat.json"), "w") as f:
        json.dump({"source": "tests/unit/test_native_forward.cpp:7706-7930 input patterns",
                   "cases": kat_cases()}, f, indent=0)
    arrs = {}
    for qtype, K, N, M in ((Q4_K, 512, 6, 3), (Q6_K, 512, 6, 3), (Q8_0, 96, 6, 3)):
        w = synth.blocks(qtype, N, K, seed=100 + qtype)
        x = synth.activations(M, K, seed=200 + qtype, outlier_frac=0.05)
        a, _, _ = q8_1_numpy(x)
        arrs[f"w_{qtype}"] = w
        arrs[f"x_{qtype}"] = x
        arrs[f"a_{qtype}"] = a
        arrs[f"wf_{qtype}"] = dequant_f32(qtype, w, N, K)
        arrs[f"y_{qtype}"] = qref.act_f64(a, M, K) @ qref.dequant_f64(qtype, w, N, K).T
    arrs["dr_x"], arrs["dr_q8_1"] = double_rounding_blocks()
    np.savez_compressed(os.path.join(HERE, "gemv_small.npz"), **arrs)
    print("wrote", os.listdir(HERE))


if __name__ == "__main__":
    main()
