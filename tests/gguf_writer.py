"""Minimal GGUF v2/v3 writer for the loader tests (test infrastructure).

Follows the published GGUF layout (ggml docs/gguf.md, the format the
reference's loader reads, gguf_model_loader.cpp:351-901): header
{magic, u32 version, i64 n_tensors, i64 n_kv}, the key/value pairs
{u64-length key, u32 type, value}, the tensor infos {name, u32 n_dims,
i64 ne[n_dims], u32 type, u64 offset}, zero padding to `general.alignment`
(default 32), then the tensor bytes at their offsets.  Every field can be
overridden so the tests can build the malformed files the loader rejects.
"""
import struct

import numpy as np

U8, I8, U16, I16, U32, I32, F32, BOOL, STRING, ARRAY, U64, I64, F64 = range(13)
_FMT = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<?",
        U64: "<Q", I64: "<q", F64: "<d"}


def enc_string(s):
    b = s.encode() if isinstance(s, str) else bytes(s)
    return struct.pack("<Q", len(b)) + b


def enc_value(vtype, value):
    if vtype in _FMT:
        return struct.pack(_FMT[vtype], value)
    if vtype == STRING:
        return enc_string(value)
    if vtype == ARRAY:
        etype, items = value
        out = struct.pack("<IQ", etype, len(items))
        return out + b"".join(enc_value(etype, v) for v in items)
    raise ValueError(vtype)


def enc_kv(key, vtype, value):
    return enc_string(key) + struct.pack("<I", vtype) + enc_value(vtype, value)


def enc_tensor_info(name, qtype, shape, offset):
    out = enc_string(name) + struct.pack("<I", len(shape))
    out += b"".join(struct.pack("<q", d) for d in shape)
    return out + struct.pack("<IQ", qtype, offset)


def build(kvs=(), tensors=(), version=3, magic=b"GGUF", n_tensors=None, n_kv=None,
          alignment=None, offsets=None, raw_kv=None, raw_infos=None):
    """kvs: [(key, type, value)]; tensors: [(name, qtype, shape ne0-first, bytes)].
    Returns (file bytes, [data-section offset of each tensor])."""
    kv_blob = raw_kv if raw_kv is not None else b"".join(enc_kv(*kv) for kv in kvs)
    align = alignment or 32
    offs, pos = [], 0
    for _, _, _, data in tensors:
        pos = (pos + align - 1) // align * align
        offs.append(pos)
        pos += len(data)
    if offsets is not None:
        offs = list(offsets)
    if raw_infos is not None:
        info_blob = raw_infos
    else:
        info_blob = b"".join(enc_tensor_info(n, q, s, o) for (n, q, s, _), o in zip(tensors, offs))
    head = magic + struct.pack("<Iqq", version,
                               len(tensors) if n_tensors is None else n_tensors,
                               len(kvs) if n_kv is None else n_kv)
    meta = head + kv_blob + info_blob
    data_start = (len(meta) + align - 1) // align * align
    out = bytearray(meta + b"\0" * (data_start - len(meta)))
    end = data_start + (max((o + len(d) for o, (_, _, _, d) in zip(offs, tensors)), default=0))
    out.extend(b"\0" * (end - len(out)))
    for o, (_, _, _, d) in zip(offs, tensors):
        out[data_start + o:data_start + o + len(d)] = bytes(d)
    return bytes(out), offs


def write(path, **kw):
    data, offs = build(**kw)
    with open(path, "wb") as f:
        f.write(data)
    return offs


def random_bytes(n, seed):
    return np.random.default_rng(seed).integers(0, 256, n, dtype=np.uint8).tobytes()
