"""GGUF weight files through the C ABI of include/ifx_gguf.h.

`GGUFFile` parses and maps a file (the reference's GGUFModelLoader::Load,
runtime/backends/cuda/native/gguf_model_loader.cpp:284-349); `upload` puts
every tensor into one device buffer at 256-byte aligned offsets
(UploadToGPU, :1005-1047) and returns per-tensor device views that the
GEMV/GEMM entry points take as W.  `layer_weights` resolves the per-layer
projection names the reference's QuantizedWeightMap uses
(quantized_weight_map.cpp:379-434, tied LM head at :81-86).
"""
import ctypes
from dataclasses import dataclass

import numpy as np

from . import _lib

VALUE_DTYPES = {0: np.uint8, 1: np.int8, 2: np.uint16, 3: np.int16, 4: np.uint32, 5: np.int32,
                6: np.float32, 7: np.bool_, 10: np.uint64, 11: np.int64, 12: np.float64}
INT_TYPES = {0, 1, 2, 3, 4, 5, 7, 10, 11}
STRING, ARRAY = 8, 9

# Per-layer projection -> GGUF component name (gguf_util.cpp:286-305).
PROJECTIONS = {"q": "attn_q", "k": "attn_k", "v": "attn_v", "o": "attn_output",
               "gate": "ffn_gate", "up": "ffn_up", "down": "ffn_down"}


class GGUFError(RuntimeError):
    def __init__(self, status, what=""):
        lib = _lib.load()
        msg = lib.ifx_gguf_status_string(status).decode()
        super().__init__(f"{what}: {msg} (status {status})" if what else msg)
        self.status = status


@dataclass
class TensorInfo:
    index: int
    name: str
    type: int
    shape: tuple      # ne[0] first (innermost), as stored
    offset: int       # in the data section
    byte_size: int

    @property
    def rows(self):
        """N of a weight matrix [N][K] (ne[1..] folded)."""
        return int(np.prod(self.shape[1:])) if len(self.shape) > 1 else 1

    @property
    def cols(self):
        return int(self.shape[0])


def tensor_bytes(qtype, shape):
    lib = _lib.load()
    arr = (ctypes.c_int64 * len(shape))(*shape)
    return int(lib.ifx_gguf_tensor_bytes(qtype, arr, len(shape)))


def type_name(qtype):
    return _lib.load().ifx_gguf_type_name(qtype).decode()


def parse_name(name):
    """-> (layer, component, kind) as gguf_util.cpp:218-268."""
    lib = _lib.load()
    layer = ctypes.c_int(0)
    comp, kind = ctypes.create_string_buffer(128), ctypes.create_string_buffer(64)
    rc = lib.ifx_gguf_parse_name(name.encode(), ctypes.byref(layer), comp, 128, kind, 64)
    if rc:
        raise GGUFError(rc, name)
    return layer.value, comp.value.decode(), kind.value.decode()


class GGUFFile:
    def __init__(self, path):
        self._lib = _lib.load()
        self._h = ctypes.c_void_p()
        rc = self._lib.ifx_gguf_open(str(path).encode(), ctypes.byref(self._h))
        if rc:
            raise GGUFError(rc, str(path))
        self.path = str(path)
        n = self._lib.ifx_gguf_n_tensors(self._h)
        self.tensors = []
        info = _lib.GgufTensor()
        for i in range(n):
            rc = self._lib.ifx_gguf_tensor_info(self._h, i, ctypes.byref(info))
            if rc:
                raise GGUFError(rc, f"tensor {i}")
            self.tensors.append(TensorInfo(i, info.name.decode(), info.type,
                                           tuple(info.shape[:info.n_dims]), info.offset,
                                           info.byte_size))
        self._by_name = {t.name: t for t in self.tensors}

    # ------------------------------------------------------------ lifetime
    def close(self):
        if self._h:
            self._lib.ifx_gguf_close(self._h)
            self._h = ctypes.c_void_p()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    # -------------------------------------------------------------- header
    @property
    def version(self):
        return self._lib.ifx_gguf_version(self._h)

    @property
    def alignment(self):
        return self._lib.ifx_gguf_alignment(self._h)

    @property
    def data_offset(self):
        return self._lib.ifx_gguf_data_offset(self._h)

    # ------------------------------------------------------------- tensors
    def tensor(self, name):
        t = self._by_name.get(name)
        if t is None:
            raise KeyError(name)
        return t

    def __contains__(self, name):
        return name in self._by_name

    def host_bytes(self, name):
        """A copy of the tensor's raw bytes (uint8)."""
        t = self.tensor(name)
        info = _lib.GgufTensor()
        rc = self._lib.ifx_gguf_tensor_info(self._h, t.index, ctypes.byref(info))
        if rc:
            raise GGUFError(rc, name)
        buf = (ctypes.c_uint8 * t.byte_size).from_address(info.host_data)
        return np.frombuffer(buf, dtype=np.uint8).copy()

    # ------------------------------------------------------------ metadata
    def keys(self):
        out = []
        key, vt = ctypes.c_char_p(), ctypes.c_int()
        for i in range(self._lib.ifx_gguf_n_kv(self._h)):
            self._lib.ifx_gguf_kv_key(self._h, i, ctypes.byref(key), ctypes.byref(vt))
            out.append((key.value.decode(), vt.value))
        return out

    def get(self, key, default=None):
        types = dict(self.keys())
        if key not in types:
            return default
        vt, k = types[key], key.encode()
        if vt in INT_TYPES:
            v = ctypes.c_int64()
            rc = self._lib.ifx_gguf_get_int(self._h, k, ctypes.byref(v))
            if rc:
                raise GGUFError(rc, key)
            return bool(v.value) if vt == 7 else v.value
        if vt in (6, 12):
            v = ctypes.c_double()
            rc = self._lib.ifx_gguf_get_float(self._h, k, ctypes.byref(v))
            if rc:
                raise GGUFError(rc, key)
            return v.value
        if vt == STRING:
            p, n = ctypes.c_void_p(), ctypes.c_uint64()
            rc = self._lib.ifx_gguf_get_string(self._h, k, ctypes.byref(p), ctypes.byref(n))
            if rc:
                raise GGUFError(rc, key)
            return ctypes.string_at(p, n.value).decode("utf-8", "replace")
        et, cnt = ctypes.c_int(), ctypes.c_uint64()
        rc = self._lib.ifx_gguf_get_array(self._h, k, ctypes.byref(et), ctypes.byref(cnt))
        if rc:
            raise GGUFError(rc, key)
        if et.value == STRING:
            out = []
            p, n = ctypes.c_void_p(), ctypes.c_uint64()
            for i in range(cnt.value):
                rc = self._lib.ifx_gguf_get_array_string(self._h, k, i, ctypes.byref(p),
                                                         ctypes.byref(n))
                if rc:
                    raise GGUFError(rc, f"{key}[{i}]")
                out.append(ctypes.string_at(p, n.value).decode("utf-8", "replace"))
            return out
        p = ctypes.c_void_p()
        rc = self._lib.ifx_gguf_get_array_data(self._h, k, ctypes.byref(p), ctypes.byref(et),
                                               ctypes.byref(cnt))
        if rc:
            raise GGUFError(rc, key)
        dt = np.dtype(VALUE_DTYPES[et.value])
        if cnt.value == 0:
            return np.zeros(0, dt)
        raw = ctypes.string_at(p, cnt.value * dt.itemsize)
        return np.frombuffer(raw, dtype=dt).copy()

    def model_info(self):
        """The hyperparameters the reference reads (gguf_model_loader.cpp:
        529-604, 903-985): keys `<arch>.*`, defaults as the reference."""
        arch = self.get("general.architecture", "")
        g = lambda k, d=0: self.get(f"{arch}.{k}", d)  # noqa: E731
        info = {"architecture": arch, "num_hidden_layers": g("block_count"),
                "hidden_size": g("embedding_length"),
                "intermediate_size": g("feed_forward_length"),
                "num_attention_heads": g("attention.head_count"),
                "num_key_value_heads": g("attention.head_count_kv"),
                "max_position_embeddings": g("context_length"),
                "rope_freq_base": g("rope.freq_base", 0.0),
                "rms_norm_eps": g("attention.layer_norm_rms_epsilon", 0.0)}
        if info["num_key_value_heads"] <= 0:
            info["num_key_value_heads"] = info["num_attention_heads"]
        if info["rms_norm_eps"] <= 0:
            info["rms_norm_eps"] = 1e-6
        emb = self._by_name.get("token_embd.weight") or self._by_name.get("tok_emb.weight")
        info["vocab_size"] = 0
        if emb is not None and len(emb.shape) >= 2:
            info["vocab_size"] = max(emb.shape[:2])
            if info["hidden_size"] <= 0:
                info["hidden_size"] = min(emb.shape[:2])
        elif emb is not None:
            info["vocab_size"] = emb.shape[0]
        return info

    # -------------------------------------------------------------- upload
    def device_bytes(self, align=256):
        return int(self._lib.ifx_gguf_device_bytes(self._h, align))

    def upload(self, device="cuda", align=256):
        """-> (buffer, {name: uint8 device view of that tensor's bytes})."""
        import torch
        n = self.device_bytes(align)
        buf = torch.empty(max(n, align), dtype=torch.uint8, device=device)
        offs = (ctypes.c_uint64 * max(1, len(self.tensors)))()
        stream = torch.cuda.current_stream(buf.device).cuda_stream
        rc = self._lib.ifx_gguf_upload(self._h, ctypes.c_void_p(buf.data_ptr()), buf.numel(),
                                       align, offs, ctypes.c_void_p(stream))
        if rc:
            raise GGUFError(rc, "upload")
        views = {t.name: buf[offs[t.index]:offs[t.index] + t.byte_size] for t in self.tensors}
        return buf, views

    def layer_weights(self, views, layer):
        """{proj: (quant type, N, K, device view)} of one block."""
        out = {}
        for proj, comp in PROJECTIONS.items():
            name = f"blk.{layer}.{comp}.weight"
            if name in self._by_name:
                t = self._by_name[name]
                out[proj] = (t.type, t.rows, t.cols, views[name])
        return out

    def lm_head(self, views):
        """(type, N, K, view) of output.weight, tied to the token embeddings
        when the file has none (quantized_weight_map.cpp:81-86)."""
        for name in ("output.weight", "token_embd.weight", "tok_emb.weight"):
            if name in self._by_name:
                t = self._by_name[name]
                return t.type, t.rows, t.cols, views[name]
        return None
