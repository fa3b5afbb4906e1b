"""Independent numpy statements of the GGUF formats and the deterministic
input patterns of the reference's own tests, used to pin the oracle.

Written from the block format descriptions, vectorised, in float64, so a
mistake in the oracle's per-element loops (an index, a nibble, a sign)
shows up as a mismatch here rather than being copied.
"""
import numpy as np

Q8_0, Q8_1, Q4_K, Q5_K, Q6_K, Q8_K = 8, 9, 12, 13, 14, 15


def f16(bytes2):
    return np.ascontiguousarray(bytes2).view(np.float16).astype(np.float64)[..., 0]


def pack_scale_min_k4(sc, m):
    """Inverse of get_scale_min_k4: 8 six-bit scales and mins -> 12 bytes.
    Bytes 0-3 carry sc[0..3] plus the top 2 bits of sc[4..7]; bytes 4-7 carry
    m[0..3] plus the top 2 bits of m[4..7]; bytes 8-11 carry the low nibbles
    of sc[4..7] (low) and m[4..7] (high)."""
    sc = np.asarray(sc, np.uint32)
    m = np.asarray(m, np.uint32)
    q = np.zeros(sc.shape[:-1] + (12,), np.uint32)
    for j in range(4):
        q[..., j] = sc[..., j] | ((sc[..., j + 4] >> 4) << 6)
        q[..., j + 4] = m[..., j] | ((m[..., j + 4] >> 4) << 6)
        q[..., j + 8] = (sc[..., j + 4] & 0xF) | ((m[..., j + 4] & 0xF) << 4)
    return q.astype(np.uint8)


def unpack_scale_min_k4(q):
    """Vectorised (all 8 sub-blocks at once) 12 bytes -> (sc[8], m[8])."""
    q = np.asarray(q, np.int64)
    sc = np.empty(q.shape[:-1] + (8,), np.int64)
    m = np.empty_like(sc)
    sc[..., :4] = q[..., 0:4] & 63
    m[..., :4] = q[..., 4:8] & 63
    sc[..., 4:] = (q[..., 8:12] & 0xF) | ((q[..., 0:4] >> 6) << 4)
    m[..., 4:] = (q[..., 8:12] >> 4) | ((q[..., 4:8] >> 6) << 4)
    return sc, m


def dequant_f64(qtype, w, n_rows, K):
    """Exact dequantized weights in float64, [n_rows, K]."""
    if qtype == Q4_K:
        b = w.reshape(-1, 144)
        d, dmin = f16(b[:, 0:2]), f16(b[:, 2:4])
        sc, m = unpack_scale_min_k4(b[:, 4:16])
        qs = b[:, 16:144].reshape(-1, 4, 32).astype(np.int64)
        q = np.stack([qs & 0xF, qs >> 4], axis=2).reshape(-1, 8, 32)  # sub-block 2p, 2p+1
        out = d[:, None, None] * sc[:, :, None] * q - dmin[:, None, None] * m[:, :, None]
    elif qtype == Q6_K:
        b = w.reshape(-1, 210)
        ql = b[:, 0:128].reshape(-1, 2, 2, 32).astype(np.int64)   # g, half, e
        qh = b[:, 128:192].reshape(-1, 2, 32).astype(np.int64)    # g, e
        sc = b[:, 192:208].view(np.int8).astype(np.int64).reshape(-1, 2, 4, 2)  # g, sub, e/16
        d = f16(b[:, 208:210])
        lo = np.stack([ql[:, :, 0] & 0xF, ql[:, :, 1] & 0xF, ql[:, :, 0] >> 4, ql[:, :, 1] >> 4], 2)
        hi = np.stack([(qh >> (2 * s)) & 3 for s in range(4)], 2)
        q = (lo | (hi << 4)) - 32                                   # [nb, g, sub, 32]
        scale = np.repeat(sc, 16, axis=3)                           # [nb, g, sub, 32]
        out = d[:, None, None, None] * scale * q
    elif qtype == Q8_0:
        b = w.reshape(-1, 34)
        out = f16(b[:, 0:2])[:, None] * b[:, 2:34].view(np.int8).astype(np.float64)
    elif qtype == Q5_K:
        # Q4_K's nibbles plus a fifth bit: bit j of qh[e] belongs to value e
        # of sub-block j (qh[32] precedes qs[128] in the block)
        b = w.reshape(-1, 176)
        d, dmin = f16(b[:, 0:2]), f16(b[:, 2:4])
        sc, m = unpack_scale_min_k4(b[:, 4:16])
        qh = b[:, 16:48].astype(np.int64)                           # [nb, e]
        qs = b[:, 48:176].reshape(-1, 4, 32).astype(np.int64)
        q = np.stack([qs & 0xF, qs >> 4], axis=2).reshape(-1, 8, 32)
        q = q + 16 * ((qh[:, None, :] >> np.arange(8)[None, :, None]) & 1)
        out = d[:, None, None] * sc[:, :, None] * q - dmin[:, None, None] * m[:, :, None]
    elif qtype == Q8_K:
        b = w.reshape(-1, 292)
        d = np.ascontiguousarray(b[:, 0:4]).view(np.float32).astype(np.float64)[:, 0]
        out = d[:, None] * b[:, 4:260].view(np.int8).astype(np.float64)
    else:
        raise ValueError(qtype)
    return out.reshape(n_rows, K)


def act_f64(a, M, K):
    b = a.reshape(-1, 36)
    return (f16(b[:, 0:2])[:, None] * b[:, 4:36].view(np.int8).astype(np.float64)).reshape(M, K)


def q8_1_fields(a, M, K):
    b = a.reshape(M, K // 32, 36)
    d = b[..., 0:2].copy().view(np.float16)[..., 0]
    s = b[..., 2:4].copy().view(np.float16)[..., 0]
    q = b[..., 4:36].view(np.int8)
    return d, s, q


# --- deterministic input generators of the reference's tests -------------
def enc_half(v):
    return np.array([v], np.float32).astype(np.float16).view(np.uint8)


def fill_quantized_rows(qtype, rows, blocks_per_row):
    """tests/unit/test_native_forward.cpp:112-160 (FillQuantizedRows)."""
    if qtype == Q4_K:
        out = np.zeros((rows, blocks_per_row, 144), np.uint8)
        for r in range(rows):
            for k in range(blocks_per_row):
                out[r, k, 0:2] = enc_half(0.012 * (((r + k) % 5) + 1))
                out[r, k, 2:4] = enc_half(0.006 * (((r + k) % 3) + 1))
                out[r, k, 4:16] = [(r * 17 + k * 7 + i * 5) & 0xFF for i in range(12)]
                out[r, k, 16:144] = [(r * 13 + k * 11 + i * 3) & 0xFF for i in range(128)]
        return out.reshape(rows, -1)
    out = np.zeros((rows, blocks_per_row, 210), np.uint8)
    for r in range(rows):
        for k in range(blocks_per_row):
            out[r, k, 0:128] = [(r * 11 + k * 5 + i * 3) & 0xFF for i in range(128)]
            out[r, k, 128:192] = [(r * 7 + k * 13 + i * 9) & 0xFF for i in range(64)]
            out[r, k, 192:208] = np.array([((r * 5 + k * 3 + i * 7) % 31) - 15 for i in range(16)],
                                          np.int8).view(np.uint8)
            out[r, k, 208:210] = enc_half(0.01 * (((r + k) % 5) + 1))
    return out.reshape(rows, -1)


def make_q4_rows(rows, blocks_per_row, seed):
    """tests/unit/test_native_rowpair_kernels.cpp:42-64 (MakeQ4Rows)."""
    out = np.zeros((rows, blocks_per_row, 144), np.uint8)
    for r in range(rows):
        for k in range(blocks_per_row):
            out[r, k, 0:2] = enc_half(0.02 * (((r + k + seed) % 4) + 1))
            out[r, k, 2:4] = enc_half(0.01 * (((r + k + seed) % 3) + 1))
            out[r, k, 4:16] = [(seed * 17 + r * 7 + k * 11 + i * 5) & 0xFF for i in range(12)]
            out[r, k, 16:144] = [(seed * 11 + r * 13 + k * 19 + i * 3) & 0xFF for i in range(128)]
    return out.reshape(rows, -1)


def make_wave_tensor(count, scale, bias=0.0):
    """tests/unit/test_native_forward.cpp:47-55 (MakeWaveTensor), fp16."""
    i = np.arange(count, dtype=np.float32)
    return (np.float32(bias) + np.float32(scale) * np.sin(np.float32(0.173) * i + np.float32(0.031))
            ).astype(np.float16)
