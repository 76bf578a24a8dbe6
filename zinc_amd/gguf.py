"""GGUF model files: reading (the native parser in libzinc_hip.so, which
restates src/model/gguf.zig and loader.zig's extractConfig) and writing.

    f = GGUFFile(path)              # gguf.parse over an mmap (loader.zig:420-445)
    f.get_u32("qwen3.block_count")  # GGUFFile.getU32 (gguf.zig:278-282), None when absent
    f.find_tensor("token_embd.weight")
    f.model_config(max_ctx=8192)    # extractConfig -> zh_model_config fields
    eng = InferenceEngine.from_gguf(ctx, path, max_ctx)   # loader.load + init

write_gguf() writes a GGUF v3 file (little-endian, tensor data aligned to
general.alignment); export_engine() writes an engine's weights under
llama.cpp's tensor names and qwen3 / qwen3moe metadata, so a model built in
this package can be loaded back like a downloaded one.
"""
import ctypes as C
import struct

import numpy as np

from .hip import ModelConfig, ZincError, lib

MAGIC = 0x46554747
# GGUFType tags (gguf.zig:20-35)
U8, I8, U16, I16, U32, I32, F32, BOOL, STRING, ARRAY, U64, I64, F64 = range(13)
_SCALAR = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<B",
           U64: "<Q", I64: "<q", F64: "<d"}
# GGML block geometry (gguf.zig:75-124): type -> (elements per block, bytes per block)
GGML_BLOCK = {0: (1, 4), 1: (1, 2), 30: (1, 2), 28: (1, 8), 24: (1, 1), 25: (1, 2), 26: (1, 4), 27: (1, 8),
              2: (32, 18), 3: (32, 20), 6: (32, 22), 7: (32, 24), 8: (32, 34), 9: (32, 36), 39: (32, 17),
              10: (256, 84), 11: (256, 110), 12: (256, 144), 13: (256, 176), 14: (256, 210), 15: (256, 292)}


def ggml_size_bytes(ggml_type, dims):
    """TensorInfo.sizeBytes (gguf.zig:222-229): whole blocks of the element count."""
    n = 1
    for d in dims:
        n *= int(d)
    bs, bpb = GGML_BLOCK.get(int(ggml_type), (1, 0))
    return (n + bs - 1) // bs * bpb


class GGUFFile:
    """A parsed GGUF file (the native zh_gguf handle over a read-only mmap)."""

    def __init__(self, path):
        self.h = None
        h = C.c_void_p()
        rc = lib().zh_gguf_open(str(path).encode(), C.byref(h))
        if rc:
            raise ZincError(rc, lib().zh_gguf_last_error(None).decode())
        self.h = h
        self.path = str(path)

    def close(self):
        if self.h:
            lib().zh_gguf_close(self.h)
            self.h = None

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    def __del__(self):
        self.close()

    @property
    def version(self):
        return lib().zh_gguf_version(self.h)

    @property
    def tensor_data_offset(self):
        return lib().zh_gguf_data_offset(self.h)

    def tensors(self):
        """[(name, dims, ggml_type, offset, size_bytes)] in file order."""
        out = []
        for i in range(lib().zh_gguf_tensor_count(self.h)):
            name, nd, t, off, nb = C.c_char_p(), C.c_uint32(), C.c_uint32(), C.c_uint64(), C.c_uint64()
            dims = (C.c_uint64 * 4)()
            lib().zh_gguf_tensor_info(self.h, i, C.byref(name), C.byref(nd), dims, C.byref(t), C.byref(off),
                                      C.byref(nb))
            out.append((name.value.decode(), [dims[d] for d in range(nd.value)], t.value, off.value, nb.value))
        return out

    def find_tensor(self, name):
        """findTensor (gguf.zig:305-310): (name, dims, type, offset, bytes) or None."""
        i = lib().zh_gguf_find_tensor(self.h, name.encode())
        return None if i < 0 else self.tensors()[i]

    def metadata(self):
        """[(key, type, elem_type, count)] in file order."""
        out = []
        for i in range(lib().zh_gguf_metadata_count(self.h)):
            k, t, e, n = C.c_char_p(), C.c_uint32(), C.c_uint32(), C.c_uint64()
            lib().zh_gguf_metadata_entry(self.h, i, C.byref(k), C.byref(t), C.byref(e), C.byref(n))
            out.append((k.value.decode(), t.value, e.value, n.value))
        return out

    def _get(self, fn, ctype, key):
        v = ctype()
        return v.value if fn(self.h, key.encode(), C.byref(v)) == 0 else None

    def get_u32(self, key):
        return self._get(lib().zh_gguf_get_u32, C.c_uint32, key)

    def get_u64(self, key):
        return self._get(lib().zh_gguf_get_u64, C.c_uint64, key)

    def get_f32(self, key):
        return self._get(lib().zh_gguf_get_f32, C.c_float, key)

    def get_bool(self, key):
        v = self._get(lib().zh_gguf_get_bool, C.c_int, key)
        return None if v is None else bool(v)

    def get_string(self, key):
        s, n = C.c_char_p(), C.c_uint64()
        if lib().zh_gguf_get_string(self.h, key.encode(), C.byref(s), C.byref(n)):
            return None
        return C.string_at(s, n.value).decode()

    def model_config(self, max_ctx=0):
        """extractConfig (loader.zig:81-346) as zh_model_config fields."""
        c = ModelConfig()
        rc = lib().zh_gguf_model_config(self.h, max_ctx, C.byref(c))
        if rc:
            raise ZincError(rc, lib().zh_gguf_last_error(self.h).decode())
        return {name: getattr(c, name) for name, _ in ModelConfig._fields_ if name != "reserved"}


# ---------------------------------------------------------------------------
# writing
# ---------------------------------------------------------------------------
def _tag_of(v):
    if isinstance(v, bool):
        return BOOL
    if isinstance(v, int):
        return U32 if 0 <= v < 2**32 else I64
    if isinstance(v, float):
        return F32
    if isinstance(v, str):
        return STRING
    raise TypeError(f"cannot infer a GGUF type for {v!r}; pass (tag, value)")


def _pack_value(tag, v):
    if tag == STRING:
        b = v.encode() if isinstance(v, str) else bytes(v)
        return struct.pack("<Q", len(b)) + b
    if tag == ARRAY:
        etag, items = v
        return struct.pack("<IQ", etag, len(items)) + b"".join(_pack_value(etag, x) for x in items)
    if tag == BOOL:
        return struct.pack("<B", 1 if v else 0)
    return struct.pack(_SCALAR[tag], v)


def write_gguf(path, metadata, tensors, alignment=32, version=3):
    """Write a GGUF file.

    metadata: [(key, value)] or [(key, (tag, value))]; an array value is
    (ARRAY, (elem_tag, [items])). tensors: [(name, dims, ggml_type, data)]
    with dims in ggml order (dims[0] contiguous) and data a bytes-like or
    numpy array of exactly ggml_size_bytes(type, dims) bytes. Each tensor's
    data starts on an `alignment` boundary of the data section."""
    meta = list(metadata)
    if alignment != 32 and not any(k == "general.alignment" for k, _ in meta):
        meta.append(("general.alignment", (U32, alignment)))
    head = bytearray(struct.pack("<IIQQ", MAGIC, version, len(tensors), len(meta)))
    for k, v in meta:
        tag, val = v if isinstance(v, tuple) and len(v) == 2 and isinstance(v[0], int) and not isinstance(v[0], bool) \
            else (_tag_of(v), v)
        head += _pack_value(STRING, k) + struct.pack("<I", tag) + _pack_value(tag, val)
    off = 0
    offsets = []
    for name, dims, t, data in tensors:
        nb = ggml_size_bytes(t, dims)
        if len(memoryview(data).cast("B")) != nb:
            raise ValueError(f"{name}: {len(memoryview(data).cast('B'))} bytes, expected {nb}")
        offsets.append(off)
        head += _pack_value(STRING, name) + struct.pack("<I", len(dims))
        head += b"".join(struct.pack("<Q", int(d)) for d in dims) + struct.pack("<IQ", t, off)
        off = (off + nb + alignment - 1) // alignment * alignment
    with open(path, "wb") as fh:
        fh.write(head)
        fh.write(b"\0" * ((-len(head)) % alignment))
        pos = 0
        for (name, dims, t, data), o in zip(tensors, offsets):
            fh.write(b"\0" * (o - pos))
            mv = memoryview(data).cast("B")
            fh.write(mv)
            pos = o + len(mv)


# engine stream ids (include/zinc_hip.h zh_engine_tensor) and GGUF names
_KINDS = {1: "attn_norm", 2: "attn_q", 3: "attn_k", 4: "attn_v", 5: "attn_output", 6: "attn_q_norm",
          7: "attn_k_norm", 8: "ffn_norm", 9: "ffn_gate", 10: "ffn_up", 11: "ffn_down", 12: "ffn_gate_inp",
          13: "ffn_gate_exps", 14: "ffn_up_exps", 15: "ffn_down_exps"}


def engine_tensor_list(cfg, tied=False):
    """[(stream, gguf name, ggml dims)] of a model config, in llama.cpp's order."""
    H, hd, V = cfg["hidden"], cfg["head_dim"], cfg["vocab"]
    qd, kvd = cfg["n_heads"] * hd, cfg["n_kv_heads"] * hd
    out = [(1, "token_embd.weight", [H, V]), (2, "output_norm.weight", [H])]
    if not tied:
        out.append((3, "output.weight", [H, V]))
    E, F = cfg.get("n_experts", 0), cfg.get("expert_ffn", 0)
    for l in range(cfg["n_layers"]):
        dims = {1: [H], 2: [H, qd], 3: [H, kvd], 4: [H, kvd], 5: [qd, H], 6: [hd], 7: [hd], 8: [H]}
        if E == 0:
            dims.update({9: [H, cfg["ffn"]], 10: [H, cfg["ffn"]], 11: [cfg["ffn"], H]})
        else:
            dims.update({12: [H, E], 13: [H, F, E], 14: [H, F, E], 15: [F, H, E]})
        for kind, d in dims.items():
            out.append((((l + 1) << 8) | kind, f"blk.{l}.{_KINDS[kind]}.weight", d))
    return out


def export_engine(engine, path, arch=None, tied=False, extra_metadata=()):
    """Write the weights of an InferenceEngine as a GGUF file with qwen3 /
    qwen3moe metadata (the keys extractConfig reads). tied=True omits
    output.weight (the LM head then reads token_embd.weight)."""
    cfg = engine.config
    moe = cfg.get("n_experts", 0) > 0
    arch = arch or ("qwen3moe" if moe else "qwen3")
    p = arch + "."
    meta = [("general.architecture", arch), ("general.alignment", (U32, 32)),
            (p + "block_count", (U32, cfg["n_layers"])), (p + "context_length", (U32, cfg["max_ctx"])),
            (p + "embedding_length", (U32, cfg["hidden"])),
            (p + "attention.head_count", (U32, cfg["n_heads"])),
            (p + "attention.head_count_kv", (U32, cfg["n_kv_heads"])),
            (p + "attention.key_length", (U32, cfg["head_dim"])),
            (p + "attention.value_length", (U32, cfg["head_dim"])),
            (p + "rope.freq_base", (F32, float(cfg["rope_base"]))),
            (p + "attention.layer_norm_rms_epsilon", (F32, float(cfg["eps"])))]
    if moe:
        meta += [(p + "expert_count", (U32, cfg["n_experts"])), (p + "expert_used_count", (U32, cfg["n_experts_used"])),
                 (p + "expert_feed_forward_length", (U32, cfg["expert_ffn"]))]
    else:
        meta.append((p + "feed_forward_length", (U32, cfg["ffn"])))
    meta += list(extra_metadata)
    tensors = []
    for stream, name, dims in engine_tensor_list(cfg, tied):
        tensors.append((name, dims, engine.tensor_type(stream), engine.tensor_bytes(stream)))
    write_gguf(path, meta, tensors)
    return path
