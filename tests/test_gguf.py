"""GGUF loader (include/ifx_gguf.h): parsing, metadata, accept/reject rules
and the upload into one device buffer.

Expectations come from the reference's own tests where they exist
(tests/unit/test_gguf_parsing.cpp:105-198: type names, CalcTensorSize,
ParseTensorName; tests/unit/test_gguf_model_loader.cpp:139-176: missing
file, bad magic, unsupported version) and otherwise from the GGUF layout
the reference parses (gguf_model_loader.cpp:351-901), written here by
tests/gguf_writer.py."""
import os
import struct

import numpy as np
import pytest

import gguf_writer as gw

Q4_K, Q6_K, Q8_0, Q5_K, Q8_K, F16, F32 = 12, 14, 8, 13, 15, 1, 0


@pytest.fixture(scope="module")
def gg():
    from inferflux_amd import gguf
    return gguf


def rows_bytes(qtype, n, k):
    be, bb = {Q4_K: (256, 144), Q6_K: (256, 210), Q8_0: (32, 34), Q5_K: (256, 176),
              Q8_K: (256, 292), F16: (1, 2), F32: (1, 4)}[qtype]
    return n * (k // be) * bb


# ------------------------------------------------------------ helpers/KATs
def test_tensor_bytes_reference_kats(gg):
    # test_gguf_parsing.cpp:153-172
    assert gg.tensor_bytes(Q4_K, (256, 1)) == 144
    assert gg.tensor_bytes(Q4_K, (512, 1)) == 288
    assert gg.tensor_bytes(F16, (1024, 1)) == 2048
    assert gg.tensor_bytes(F32, (512, 1)) == 2048


def test_tensor_bytes_all_types(gg):
    # ggml block sizes (gguf_util.cpp:549-566); partial blocks round up (:548)
    per_block = {2: (32, 18), 3: (32, 20), 6: (32, 22), 7: (32, 24), 8: (32, 34), 9: (32, 36),
                 10: (256, 96), 11: (256, 110), 12: (256, 144), 13: (256, 176),
                 14: (256, 210), 15: (256, 292)}
    for t, (be, bb) in per_block.items():
        assert gg.tensor_bytes(t, (2048, 3)) == 3 * 2048 // be * bb, t
        assert gg.tensor_bytes(t, (be + 1,)) == 2 * bb, t
    for bad in (4, 5, 16, 30):
        assert gg.tensor_bytes(bad, (256,)) == 0
    assert gg.tensor_bytes(Q4_K, (0, 4)) == 0
    assert gg.tensor_bytes(Q4_K, (-256,)) == 0


def test_type_names(gg):
    # test_gguf_parsing.cpp:112-118
    assert [gg.type_name(t) for t in (0, 1, 12, 13, 14, 15, 8)] == \
        ["f32", "f16", "q4_k", "q5_k", "q6_k", "q8_k", "q8_0"]
    assert gg.type_name(4) == "unknown"


def test_parse_name_reference_kats(gg):
    # test_gguf_parsing.cpp:174-198
    assert gg.parse_name("tok_emb.weight") == (-1, "tok_emb", "weight")
    assert gg.parse_name("token_embd.weight") == (-1, "tok_emb", "weight")
    assert gg.parse_name("output.weight") == (-2, "output", "weight")
    assert gg.parse_name("blk.0.attn_q.weight") == (0, "attn_q", "weight")
    assert gg.parse_name("blk.5.ffn_gate.weight") == (5, "ffn_gate", "weight")
    assert gg.parse_name("blk.12.attn_q.bias") == (12, "attn_q", "bias")
    assert gg.parse_name("blk.3.attn_norm") == (3, "attn_norm", "weight")
    assert gg.parse_name("output_norm.weight") == (-1, "", "")


# ------------------------------------------------------------- round trip
ALL_KVS = [
    ("general.architecture", gw.STRING, "qwen2"),
    ("general.alignment", gw.U32, 64),
    ("qwen2.block_count", gw.U32, 2),
    ("qwen2.embedding_length", gw.U32, 512),
    ("qwen2.feed_forward_length", gw.U64, 1024),
    ("qwen2.attention.head_count", gw.I32, 8),
    ("qwen2.attention.head_count_kv", gw.U16, 2),
    ("qwen2.attention.layer_norm_rms_epsilon", gw.F32, 1e-5),
    ("qwen2.rope.freq_base", gw.F64, 1000000.0),
    ("qwen2.context_length", gw.I64, 32768),
    ("t.u8", gw.U8, 200), ("t.i8", gw.I8, -5), ("t.i16", gw.I16, -300), ("t.bool", gw.BOOL, True),
    ("tokenizer.ggml.tokens", gw.ARRAY, (gw.STRING, ["<s>", "hello", "", "wörld"])),
    ("tokenizer.ggml.token_type", gw.ARRAY, (gw.I32, [1, 2, 3, -4])),
    ("t.f32s", gw.ARRAY, (gw.F32, [0.5, -1.25])),
    ("t.nested", gw.ARRAY, (gw.ARRAY, [(gw.U8, [1, 2]), (gw.U8, [])])),
    ("t.empty", gw.ARRAY, (gw.U64, [])),
]


def model_tensors():
    """A 2-layer model in the reference's GGUF names, mixed quant types."""
    out = []
    spec = [("token_embd.weight", Q8_0, 512, 1000), ("output_norm.weight", F32, 512, None)]
    for l in range(2):
        spec += [(f"blk.{l}.attn_q.weight", Q4_K, 512, 512), (f"blk.{l}.attn_k.weight", Q4_K, 512, 128),
                 (f"blk.{l}.attn_v.weight", Q6_K, 512, 128), (f"blk.{l}.attn_output.weight", Q4_K, 512, 512),
                 (f"blk.{l}.ffn_gate.weight", Q4_K, 512, 1024), (f"blk.{l}.ffn_up.weight", Q4_K, 512, 1024),
                 (f"blk.{l}.ffn_down.weight", Q6_K, 1024, 512), (f"blk.{l}.attn_norm.weight", F16, 512, None)]
    from inferflux_amd import synth
    for i, (name, q, k, n) in enumerate(spec):
        shape = (k,) if n is None else (k, n)
        if q in (F16, F32):
            data = gw.random_bytes(rows_bytes(q, 1 if n is None else n, k), i)
        else:  # valid blocks (finite fp16 scales)
            data = synth.blocks(q, n, k, seed=i).tobytes()
        assert len(data) == rows_bytes(q, 1 if n is None else n, k)
        out.append((name, q, shape, data))
    return out


@pytest.fixture(scope="module")
def model_file(tmp_path_factory):
    p = tmp_path_factory.mktemp("gguf") / "model.gguf"
    tensors = model_tensors()
    offs = gw.write(p, kvs=ALL_KVS, tensors=tensors, alignment=64)
    return p, tensors, offs


def test_roundtrip_tensors(gg, model_file):
    path, tensors, offs = model_file
    with gg.GGUFFile(path) as f:
        assert f.version == 3 and f.alignment == 64
        assert f.data_offset % 64 == 0
        assert [t.name for t in f.tensors] == [t[0] for t in tensors]
        for (name, q, shape, data), off, t in zip(tensors, offs, f.tensors):
            assert (t.type, t.shape, t.offset, t.byte_size) == (q, shape, off, len(data))
            assert f.host_bytes(name).tobytes() == data
        assert f.tensor("blk.1.ffn_down.weight").rows == 512
        assert f.tensor("blk.1.ffn_down.weight").cols == 1024
        assert "blk.2.attn_q.weight" not in f


def test_roundtrip_metadata(gg, model_file):
    path, _, _ = model_file
    with gg.GGUFFile(path) as f:
        keys = dict(f.keys())
        assert keys["general.alignment"] == gw.U32 and keys["t.nested"] == gw.ARRAY
        assert f.get("general.architecture") == "qwen2"
        assert f.get("t.u8") == 200 and f.get("t.i8") == -5 and f.get("t.i16") == -300
        assert f.get("t.bool") is True
        assert f.get("qwen2.context_length") == 32768
        assert f.get("qwen2.attention.layer_norm_rms_epsilon") == pytest.approx(1e-5, rel=1e-6)
        assert f.get("qwen2.rope.freq_base") == 1e6
        assert f.get("tokenizer.ggml.tokens") == ["<s>", "hello", "", "wörld"]
        assert f.get("tokenizer.ggml.token_type").tolist() == [1, 2, 3, -4]
        assert f.get("t.f32s").tolist() == [0.5, -1.25]
        assert f.get("t.empty").size == 0
        assert f.get("missing", 7) == 7
        info = f.model_info()
        assert info == {"architecture": "qwen2", "num_hidden_layers": 2, "hidden_size": 512,
                        "intermediate_size": 1024, "num_attention_heads": 8,
                        "num_key_value_heads": 2, "max_position_embeddings": 32768,
                        "rope_freq_base": 1e6, "rms_norm_eps": pytest.approx(1e-5, rel=1e-6),
                        "vocab_size": 1000}


def test_wrong_type_getters(gg, model_file):
    import ctypes
    from inferflux_amd import _lib
    path, _, _ = model_file
    lib = _lib.load()
    with gg.GGUFFile(path) as f:
        v = ctypes.c_int64()
        assert lib.ifx_gguf_get_int(f._h, b"general.architecture", ctypes.byref(v)) == 18
        assert lib.ifx_gguf_get_int(f._h, b"nope", ctypes.byref(v)) == 17
        d = ctypes.c_double()
        assert lib.ifx_gguf_get_float(f._h, b"t.u8", ctypes.byref(d)) == 18


def test_default_alignment_and_v2(gg, tmp_path):
    # default alignment 32 (gguf_model_loader.cpp:380); version 2 accepted
    t = [("w", Q4_K, (256, 3), gw.random_bytes(3 * 144, 1)), ("b", F32, (5,), b"\1" * 20)]
    p = tmp_path / "v2.gguf"
    offs = gw.write(p, tensors=t, version=2)
    with gg.GGUFFile(p) as f:
        assert f.alignment == 32 and f.version == 2
        assert [x.offset for x in f.tensors] == offs == [0, 448]
        assert f.data_offset % 32 == 0
        assert f.host_bytes("b").tobytes() == b"\1" * 20


def test_model_without_tensors(gg, tmp_path):
    p = tmp_path / "empty.gguf"
    gw.write(p, kvs=[("general.architecture", gw.STRING, "llama")])
    with gg.GGUFFile(p) as f:
        assert f.tensors == [] and f.device_bytes() == 0
        assert f.model_info()["rms_norm_eps"] == 1e-6


def test_duplicate_tensor_name_last_wins(gg, tmp_path):
    # the reference's map assignment (gguf_model_loader.cpp:843) keeps the last
    t = [("w", F32, (4,), b"\0" * 16), ("x", F32, (2,), b"\2" * 8), ("w", F32, (8,), b"\1" * 32)]
    p = tmp_path / "dup.gguf"
    gw.write(p, tensors=t)
    with gg.GGUFFile(p) as f:
        assert [x.name for x in f.tensors] == ["w", "x"]
        assert f.tensor("w").shape == (8,) and f.host_bytes("w").tobytes() == b"\1" * 32


# ---------------------------------------------------------------- rejects
def status_of(gg, path):
    with pytest.raises(gg.GGUFError) as e:
        gg.GGUFFile(path)
    return e.value.status


def test_reject_missing_file(gg, tmp_path):
    assert status_of(gg, tmp_path / "nope.gguf") == 10  # test_gguf_model_loader.cpp:139


@pytest.mark.parametrize("kw,status", [
    (dict(magic=b"GGUX"), 11),                        # :146-159
    (dict(version=1), 12), (dict(version=0), 12),     # legacy (gguf_util.cpp:408)
    (dict(version=4), 12),                            # :161-175
    (dict(n_tensors=-1), 14), (dict(n_kv=-2), 14),    # gguf_model_loader.cpp:362
])
def test_reject_header(gg, tmp_path, kw, status):
    p = tmp_path / "bad.gguf"
    gw.write(p, **kw)
    assert status_of(gg, p) == status


def test_reject_truncation_everywhere(gg, tmp_path):
    """Cutting the file inside the header, a key, a value, an array, a tensor
    info or the data is always an error, never a crash."""
    data, _ = gw.build(kvs=ALL_KVS, tensors=model_tensors(), alignment=64)
    p = tmp_path / "cut.gguf"
    meta_end = data.index(b"token_embd.weight") + 200
    for cut in list(range(0, 64)) + list(range(64, meta_end, 7)) + [len(data) - 1]:
        p.write_bytes(data[:cut])
        assert status_of(gg, p) in (13, 16), cut


@pytest.mark.parametrize("key,vtype,value", [
    ("t.x", 13, b""),                                         # unknown value type
    ("general.alignment", gw.F32, struct.pack("<f", 32.0)),   # :432-435
    ("general.alignment", gw.U32, struct.pack("<I", 0)),      # :437
    ("general.alignment", gw.U64, struct.pack("<Q", 48)),     # :444
    ("general.architecture", gw.U32, struct.pack("<I", 1)),   # :405
    ("t.arr", gw.ARRAY, struct.pack("<IQ", 13, 1)),           # bad element type
])
def test_reject_metadata(gg, tmp_path, key, vtype, value):
    raw = gw.enc_string(key) + struct.pack("<I", vtype) + value
    p = tmp_path / "kv.gguf"
    gw.write(p, raw_kv=raw, n_kv=1)
    assert status_of(gg, p) == 14


def test_reject_oversize_string(gg, tmp_path):
    raw = struct.pack("<Q", (1 << 30) + 1) + b"k"   # gguf_util.cpp:92-96
    p = tmp_path / "s.gguf"
    gw.write(p, raw_kv=raw, n_kv=1)
    assert status_of(gg, p) == 14


@pytest.mark.parametrize("shape,qtype,status", [
    ((), Q4_K, 15), (tuple([1] * 9), F32, 15),           # :776-787
    ((256, 0), Q4_K, 15), ((256, -3), Q4_K, 15),          # :796-800
    ((256,), 16, 15), ((256,), 4, 15),                    # :811-814, size 0 (:828)
])
def test_reject_tensor_info(gg, tmp_path, shape, qtype, status):
    p = tmp_path / "t.gguf"
    info = gw.enc_tensor_info("w", qtype, shape, 0)
    gw.write(p, raw_infos=info, n_tensors=1)
    assert status_of(gg, p) == status


def test_reject_data_outside_file(gg, tmp_path):
    t = [("w", Q4_K, (256, 4), gw.random_bytes(576, 3))]
    p = tmp_path / "d.gguf"
    data, _ = gw.build(tensors=t)
    p.write_bytes(data[:-1])                      # last byte missing
    assert status_of(gg, p) == 16
    gw.write(p, raw_infos=gw.enc_tensor_info("w", Q4_K, (256, 4), 1 << 40), n_tensors=1)
    assert status_of(gg, p) == 16                 # offset far past EOF
    gw.write(p, raw_infos=gw.enc_tensor_info("w", Q4_K, (256, 4), (1 << 64) - 64), n_tensors=1)
    assert status_of(gg, p) == 16                 # offset + data start overflows


def test_device_bytes_alignment(gg, model_file):
    path, tensors, _ = model_file
    with gg.GGUFFile(path) as f:
        for align in (16, 256, 4096):
            total = 0
            for _, _, _, d in tensors:
                total = -(-total // align) * align + len(d)
            assert f.device_bytes(align) == -(-total // align) * align
        assert f.device_bytes(8) == 0 and f.device_bytes(48) == 0


# -------------------------------------------------------------- GPU upload
@pytest.mark.gpu
def test_upload_and_gemv_from_file(gg, model_file):
    """Upload every tensor into one device buffer; the views hold the file's
    bytes, and a GEMV on a loaded projection matches the oracle on the
    same bytes."""
    import torch
    from inferflux_amd import ops, synth
    from oracle import oracle as orc
    path, tensors, _ = model_file
    with gg.GGUFFile(path) as f:
        buf, views = f.upload("cuda:0", align=256)
        torch.cuda.synchronize()
        for name, _, _, data in tensors:
            assert views[name].data_ptr() % 256 == 0
            assert views[name].cpu().numpy().tobytes() == data, name
        lw = f.layer_weights(views, 1)
        assert set(lw) == {"q", "k", "v", "o", "gate", "up", "down"}
        for proj in ("gate", "down"):
            qt, N, K, w = lw[proj]
            x = synth.activations(2, K, seed=5)
            a = orc.quantize_q8_1(x)
            y = ops.qgemv(qt, w, torch.from_numpy(a).to("cuda:0"), 2, N, K).cpu().numpy()
            ye = orc.gemv_exact(qt, f.host_bytes(f"blk.1.ffn_{proj}.weight"), a, 2, N, K)
            err = np.abs(y - ye).max(axis=1)
            assert np.all(err <= 1e-3 * np.linalg.norm(ye, axis=1)), proj
        qt, N, K, w = f.lm_head(views)   # no output.weight: tied embeddings
        assert (qt, N, K) == (Q8_0, 1000, 512)


# ------------------------------------------------ C++ mirror (GgufModelLoader)
def cpp_binary():
    import subprocess
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    b = os.path.join(root, "tests", "cpp", "test_gguf_model")
    if not os.path.exists(b):
        subprocess.run(["make", "-s", "-C", os.path.join(root, "oracle")], check=True)
        subprocess.run(["make", "-s", "-C", os.path.dirname(b)], check=True)
    return b


def test_cpp_loader_cpu(model_file):
    import subprocess
    path, _, _ = model_file
    r = subprocess.run([cpp_binary(), "cpu", str(path)], capture_output=True, text=True, timeout=60)
    assert r.returncode == 0 and "cpu: 0 failure(s)" in r.stdout, r.stdout + r.stderr


@pytest.mark.gpu
def test_cpp_loader_gpu(model_file):
    import subprocess
    path, _, _ = model_file
    r = subprocess.run([cpp_binary(), "gpu", str(path)], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0 and "gpu: 0 failure(s)" in r.stdout, r.stdout + r.stderr
