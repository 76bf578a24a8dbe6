"""GGUF parsing and config extraction (CPU: host code of libzinc_hip.so).

Mirrors the reference's own tests of src/model/gguf.zig (:548-592: block
sizes, TensorInfo.sizeBytes, MetadataValue conversions) and checks the
parser on hand-assembled bytes (the GGUF v3 layout written out field by field
here, independent of zinc_amd.gguf.write_gguf), on files from the writer, and
on the failure paths parse() has (InvalidMagic, UnknownMetadataType) plus
the bounds checks it adds (TruncatedFile)."""
import struct

import numpy as np
import pytest

from zinc_amd import Q4_K, Q6_K, Q8_0, ZincError
from zinc_amd import gguf as G


def _s(x):
    b = x.encode()
    return struct.pack("<Q", len(b)) + b


def _hand_file(tmp_path, align=None):
    """A GGUF v3 file built byte by byte: 3 metadata entries, 2 tensors."""
    meta = [
        _s("general.architecture") + struct.pack("<I", 8) + _s("qwen3"),
        _s("qwen3.block_count") + struct.pack("<II", 4, 7),
        _s("tokenizer.ggml.tokens") + struct.pack("<IIQ", 9, 8, 2) + _s("a") + _s("bc"),
    ]
    if align:
        meta.append(_s("general.alignment") + struct.pack("<II", 4, align))
    tens = [
        _s("t0") + struct.pack("<I", 2) + struct.pack("<QQ", 256, 2) + struct.pack("<IQ", 12, 0),
        _s("t1") + struct.pack("<I", 1) + struct.pack("<Q", 8) + struct.pack("<IQ", 0, 288),
    ]
    head = struct.pack("<IIQQ", 0x46554747, 3, len(tens), len(meta)) + b"".join(meta) + b"".join(tens)
    a = align or 32
    pad = (-len(head)) % a
    data = bytes(range(256)) + bytes(32) + np.arange(8, dtype=np.float32).tobytes()
    p = tmp_path / "hand.gguf"
    p.write_bytes(head + bytes(pad) + data)
    return p, len(head) + pad


def test_block_sizes_and_size_bytes():
    # gguf.zig:548-582
    assert G.GGML_BLOCK[12] == (256, 144) and G.GGML_BLOCK[8] == (32, 34) and G.GGML_BLOCK[1] == (1, 2)
    assert G.ggml_size_bytes(1, [4096, 4096]) == 33554432
    assert G.ggml_size_bytes(12, [4096, 4096]) == 9437184
    assert G.ggml_size_bytes(39, [2880, 2880]) == 2880 * 90 * 17
    assert G.ggml_size_bytes(99, [10, 10]) == 0  # no geometry: 0 bytes, as the reference


@pytest.mark.parametrize("align", [None, 64])
def test_hand_assembled_file(tmp_path, align):
    p, data_off = _hand_file(tmp_path, align)
    with G.GGUFFile(p) as f:
        assert f.version == 3
        assert f.tensor_data_offset == data_off and data_off % (align or 32) == 0
        assert f.get_string("general.architecture") == "qwen3"
        assert f.get_u32("qwen3.block_count") == 7
        md = f.metadata()
        assert ("tokenizer.ggml.tokens", G.ARRAY, G.STRING, 2) in md
        ts = f.tensors()
        assert ts[0] == ("t0", [256, 2], 12, 0, 288)  # 2 Q4_K blocks
        assert ts[1] == ("t1", [8], 0, 288, 32)
        assert f.find_tensor("t1")[3] == 288 and f.find_tensor("nope") is None
        raw = p.read_bytes()
        o = f.tensor_data_offset + ts[1][3]
        assert np.array_equal(np.frombuffer(raw[o:o + 32], np.float32), np.arange(8, dtype=np.float32))


def test_metadata_conversions(tmp_path):
    # MetadataValue conversions (gguf.zig:584-592 and :143-193)
    p = tmp_path / "m.gguf"
    G.write_gguf(p, [("s", (G.STRING, "hello")), ("u32", (G.U32, 42)), ("i32n", (G.I32, -1)), ("i32", (G.I32, 5)),
                     ("u64big", (G.U64, 2**40)), ("u64", (G.U64, 9)), ("i64", (G.I64, 11)),
                     ("i64n", (G.I64, -3)), ("f32", (G.F32, 1.5)), ("f64", (G.F64, 0.25)), ("b", (G.BOOL, True)),
                     ("u32zero", (G.U32, 0)), ("u8", (G.U8, 3)), ("u16", (G.U16, 4)), ("i8", (G.I8, -2)),
                     ("i16", (G.I16, -300)), ("arr", (G.ARRAY, (G.I32, [2, 8, 4])))], [])
    with G.GGUFFile(p) as f:
        assert f.get_string("s") == "hello" and f.get_u32("s") is None
        assert f.get_u32("u32") == 42 and f.get_string("u32") is None
        assert f.get_u32("i32n") is None and f.get_u32("i32") == 5
        assert f.get_u32("u64big") is None and f.get_u64("u64big") == 2**40 and f.get_u32("u64") == 9
        assert f.get_u64("i64") == 11 and f.get_u64("i64n") is None and f.get_u32("i64") is None
        assert f.get_f32("f32") == 1.5 and f.get_f32("f64") == 0.25 and f.get_f32("u32") is None
        assert f.get_bool("b") is True and f.get_bool("u32zero") is False and f.get_bool("u8") is True
        assert f.get_bool("i32n") is True and f.get_bool("f32") is None
        # asU32 takes u32 / i32 / u64 only (gguf.zig:152-159)
        assert f.get_u32("u8") is None and f.get_u32("u16") is None
        assert f.get_u32("missing") is None
        md = {k: (t, e, n) for k, t, e, n in f.metadata()}
        assert md["arr"] == (G.ARRAY, G.I32, 3) and md["i16"] == (G.I16, 0, 1)


def test_duplicate_keys_last_wins(tmp_path):
    # the metadata map's put: a repeated key keeps the last value
    p = tmp_path / "d.gguf"
    G.write_gguf(p, [("k", (G.U32, 1)), ("k", (G.U32, 2))], [])
    with G.GGUFFile(p) as f:
        assert f.get_u32("k") == 2


def test_invalid_magic(tmp_path):
    p = tmp_path / "bad.gguf"
    p.write_bytes(b"GGUX" + bytes(20))
    with pytest.raises(ZincError) as ei:
        G.GGUFFile(p)
    assert ei.value.name == "InvalidMagic"


def test_unknown_metadata_type(tmp_path):
    head = struct.pack("<IIQQ", 0x46554747, 3, 0, 1) + _s("x") + struct.pack("<I", 13) + bytes(8)
    p = tmp_path / "u.gguf"
    p.write_bytes(head)
    with pytest.raises(ZincError) as ei:
        G.GGUFFile(p)
    assert ei.value.name == "UnknownMetadataType"
    # an array of arrays: readTypedValue has no array case (gguf.zig:519-540)
    head = struct.pack("<IIQQ", 0x46554747, 3, 0, 1) + _s("y") + struct.pack("<IIQ", 9, 9, 1) + \
        struct.pack("<IQ", 4, 0)
    p.write_bytes(head)
    with pytest.raises(ZincError) as ei:
        G.GGUFFile(p)
    assert ei.value.name == "UnknownMetadataType"
    # ... which the reference only meets for a non-empty array
    head = struct.pack("<IIQQ", 0x46554747, 3, 0, 1) + _s("z") + struct.pack("<IIQ", 9, 9, 0)
    p.write_bytes(head)
    with G.GGUFFile(p) as f:
        assert ("z", G.ARRAY, G.ARRAY, 0) in f.metadata()


def test_truncated_file(tmp_path):
    p, _ = _hand_file(tmp_path)
    raw = p.read_bytes()
    for cut in (3, 20, 40, 90, 150):
        q = tmp_path / f"t{cut}.gguf"
        q.write_bytes(raw[:cut])
        with pytest.raises(ZincError) as ei:
            G.GGUFFile(q)
        assert ei.value.name in ("TruncatedFile", "InvalidMagic"), (cut, ei.value.name)


def test_missing_file(tmp_path):
    with pytest.raises(ZincError) as ei:
        G.GGUFFile(tmp_path / "absent.gguf")
    assert ei.value.name == "IoError"


def test_writer_tensor_alignment(tmp_path):
    p = tmp_path / "w.gguf"
    a = np.arange(7, dtype=np.float32)
    b = np.arange(256 * 3, dtype=np.uint8)[:144 * 3].copy()
    G.write_gguf(p, [("general.architecture", "qwen3")], [("a", [7], 0, a), ("b", [768], Q4_K, b)], alignment=64)
    raw = p.read_bytes()
    with G.GGUFFile(p) as f:
        ts = {t[0]: t for t in f.tensors()}
        assert f.tensor_data_offset % 64 == 0 and ts["b"][3] % 64 == 0
        o = f.tensor_data_offset
        assert raw[o + ts["a"][3]:o + ts["a"][3] + 28] == a.tobytes()
        assert raw[o + ts["b"][3]:o + ts["b"][3] + ts["b"][4]] == b.tobytes()


def _qwen3_meta(arch="qwen3", **kw):
    p = arch + "."
    m = [("general.architecture", arch), (p + "block_count", (G.U32, 2)), (p + "embedding_length", (G.U32, 512)),
         (p + "attention.head_count", (G.U32, 8)), (p + "attention.head_count_kv", (G.U32, 2)),
         (p + "feed_forward_length", (G.U32, 768)), (p + "rope.freq_base", (G.F32, 1e6)),
         (p + "attention.layer_norm_rms_epsilon", (G.F32, 1e-6))]
    drop = kw.pop("drop", ())
    m = [x for x in m if x[0][len(p):] not in drop]
    m += list(kw.get("extra", []))
    return m


def test_model_config_qwen3(tmp_path):
    p = tmp_path / "c.gguf"
    emb = np.zeros(G.ggml_size_bytes(Q4_K, [512, 1000]), np.uint8)
    out = np.zeros(G.ggml_size_bytes(Q6_K, [512, 1000]), np.uint8)
    q = np.zeros(G.ggml_size_bytes(Q8_0, [512, 512]), np.uint8)
    G.write_gguf(p, _qwen3_meta(drop=("attention.key_length",)),
                 [("token_embd.weight", [512, 1000], Q4_K, emb), ("output.weight", [512, 1000], Q6_K, out),
                  ("blk.0.attn_q.weight", [512, 512], Q8_0, q)])
    with G.GGUFFile(p) as f:
        c = f.model_config(max_ctx=1000)
    assert (c["n_layers"], c["hidden"], c["n_heads"], c["n_kv_heads"]) == (2, 512, 8, 2)
    assert c["head_dim"] == 64  # key_length absent: hidden / n_heads
    assert c["ffn"] == 768 and c["n_experts"] == 0
    assert c["vocab"] == 1000  # no vocab_size: rows of output.weight
    assert c["max_ctx"] == 1008  # rounded up to 16 tokens
    assert abs(c["rope_base"] - 1e6) < 1 and abs(c["eps"] - 1e-6) < 1e-12
    assert (c["type_embd"], c["type_lm_head"], c["type_attn"]) == (Q4_K, Q6_K, Q8_0)


def test_model_config_defaults_and_rope_forms(tmp_path):
    p = tmp_path / "c2.gguf"
    meta = _qwen3_meta(drop=("attention.layer_norm_rms_epsilon", "rope.freq_base", "attention.head_count_kv"),
                       extra=[("qwen3.vocab_size", (G.U32, 320)), ("qwen3.rope.freq_base", (G.U32, 500000))])
    G.write_gguf(p, meta, [])
    with G.GGUFFile(p) as f:
        c = f.model_config()
    assert c["eps"] == pytest.approx(1e-6) and c["rope_base"] == 500000.0  # a u32 base is taken as a float
    assert c["n_kv_heads"] == 8  # head_count_kv absent: n_heads
    assert c["vocab"] == 320 and c["max_ctx"] == 4096  # context_length absent: 4096
    # an f64 base is neither form the reference reads: 10000
    G.write_gguf(p, _qwen3_meta(drop=("rope.freq_base",), extra=[("qwen3.rope.freq_base", (G.F64, 1e6))]),
                 [("token_embd.weight", [512, 64], Q4_K, np.zeros(G.ggml_size_bytes(Q4_K, [512, 64]), np.uint8))])
    with G.GGUFFile(p) as f:
        c = f.model_config()
    assert c["rope_base"] == 10000.0 and c["vocab"] == 64  # vocab from token_embd.weight


def test_model_config_moe(tmp_path):
    p = tmp_path / "m.gguf"
    meta = _qwen3_meta("qwen3moe", extra=[("qwen3moe.expert_count", (G.U32, 16)),
                                          ("qwen3moe.expert_used_count", (G.U32, 4)),
                                          ("qwen3moe.expert_feed_forward_length", (G.U32, 256)),
                                          ("qwen3moe.vocab_size", (G.U32, 100))])
    G.write_gguf(p, meta, [])
    with G.GGUFFile(p) as f:
        c = f.model_config(64)
    assert (c["n_experts"], c["n_experts_used"], c["expert_ffn"], c["ffn"]) == (16, 4, 256, 0)


@pytest.mark.parametrize("arch", ["llama", "qwen2", "gemma4", None])
def test_unsupported_architecture(tmp_path, arch):
    p = tmp_path / "a.gguf"
    meta = _qwen3_meta("qwen3")
    meta = [m for m in meta if m[0] != "general.architecture"]
    if arch:
        meta.append(("general.architecture", arch))
    G.write_gguf(p, meta, [])
    with G.GGUFFile(p) as f:
        with pytest.raises(ZincError) as ei:
            f.model_config()
    assert ei.value.name == "UnsupportedArchitecture"


def test_engine_tensor_list_names():
    from zinc_amd import DENSE_8B, MOE_48L
    names = {n for _, n, _ in G.engine_tensor_list(DENSE_8B)}
    assert {"token_embd.weight", "output.weight", "output_norm.weight", "blk.0.attn_q.weight",
            "blk.35.ffn_down.weight", "blk.3.attn_k_norm.weight"} <= names
    assert len(names) == 3 + 36 * 11
    moe = {n: d for _, n, d in G.engine_tensor_list(MOE_48L, tied=True)}
    assert "output.weight" not in moe and moe["blk.0.ffn_down_exps.weight"] == [768, 2048, 128]
