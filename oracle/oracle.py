"""ctypes bindings for the CPU parity oracle (oracle/libzinc_oracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, never by the zinc_amd product path.
"""
import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libzinc_oracle.so")

F32, F16, Q8_0, Q4_K, Q5_K, Q6_K, MXFP4 = 0, 1, 8, 12, 13, 14, 39

# Tensor stream ids shared with the HIP engine's synthetic model.
S_TOKEN_EMBD, S_OUTPUT_NORM, S_OUTPUT = 1, 2, 3
(K_ATTN_NORM, K_WQ, K_WK, K_WV, K_WO, K_Q_NORM, K_K_NORM, K_FFN_NORM,
 K_GATE, K_UP, K_DOWN, K_ROUTER, K_EXP_GATE, K_EXP_UP, K_EXP_DOWN) = range(1, 16)


def S_LAYER(layer, kind):
    return ((layer + 1) << 8) | kind


def S_KV(layer, which):
    return 0x100000 + 2 * layer + which


def build():
    subprocess.run(["make", "-s", "-C", HERE], check=True)


_lib = None


def lib():
    global _lib
    if _lib is None:
        path = os.environ.get("ZO_LIB_PATH") or LIB_PATH  # (bench.py: a -march=native build of the same source)
        if path == LIB_PATH and not os.path.exists(LIB_PATH):
            build()
        L = C.CDLL(path)
        u8p, f32p, f64p, u16p, u32p = (C.POINTER(C.c_uint8), C.POINTER(C.c_float),
                                       C.POINTER(C.c_double), C.POINTER(C.c_uint16),
                                       C.POINTER(C.c_uint32))
        sig = {
            "zo_block_size": (C.c_uint32, [C.c_uint32]),
            "zo_bytes_per_block": (C.c_uint32, [C.c_uint32]),
            "zo_tensor_bytes": (C.c_uint64, [C.c_uint32, C.c_uint64, C.c_uint64]),
            "zo_f16_to_f32": (C.c_float, [C.c_uint16]),
            "zo_f32_to_f16": (C.c_uint16, [C.c_float]),
            "zo_get_scale_min_k4": (None, [C.c_uint32, u8p, u8p, u8p]),
            "zo_dequant_row": (C.c_int, [u8p, C.c_uint32, C.c_uint32, C.c_uint32, f32p]),
            "zo_dot_q8_0_row": (C.c_float, [u8p, C.c_uint32, C.c_uint32, f32p]),
            "zo_dmmv": (C.c_int, [u8p, C.c_uint32, f32p, f32p, C.c_uint32, C.c_uint32, C.c_uint32, C.c_int]),
            "zo_dmmv_f64": (C.c_int, [u8p, C.c_uint32, f32p, f64p, C.c_uint32, C.c_uint32, C.c_int]),
            "zo_dmmv_absdot": (C.c_int, [u8p, C.c_uint32, f32p, f64p, C.c_uint32, C.c_uint32, C.c_int]),
            "zo_rms_norm_mul": (None, [f32p, f32p, C.c_uint32, f32p, C.c_uint32, C.c_uint32, C.c_float]),
            "zo_per_head_rms_norm": (None, [f32p, f32p, C.c_uint32, C.c_uint32, C.c_float]),
            "zo_rope_inv_freq": (None, [f32p, C.c_uint32, C.c_float]),
            "zo_rope": (None, [f32p, C.c_uint32, C.c_uint32, C.c_uint32, C.c_uint32, f32p]),
            "zo_swiglu": (None, [f32p, f32p, f32p, C.c_uint32]),
            "zo_attention_f16": (None, [f32p, u16p, u16p, f32p, C.c_uint32, C.c_uint32, C.c_uint32,
                                        C.c_uint32, C.c_float]),
            "zo_topk_softmax": (None, [f32p, C.c_uint32, C.c_uint32, u32p, f32p]),
            "zo_argmax": (C.c_uint32, [f32p, C.c_uint32]),
            "zo_kv_page_count": (C.c_uint32, [C.c_uint32]),
            "zo_logical_to_physical": (C.c_int64, [u32p, C.c_uint32, C.c_uint32]),
            "zo_rand": (C.c_uint64, [C.c_uint64, C.c_uint64, C.c_uint64]),
            "zo_normal": (C.c_float, [C.c_uint64]),
            "zo_synth_tensor": (C.c_int, [u8p, C.c_uint32, C.c_uint64, C.c_uint64, C.c_uint64, C.c_uint64]),
            "zo_synth_normal_f32": (None, [f32p, C.c_uint64, C.c_float, C.c_uint64, C.c_uint64]),
            "zo_synth_normal_f16": (None, [u16p, C.c_uint64, C.c_uint64, C.c_uint64]),
            "zo_synth_norm_weight": (None, [f32p, C.c_uint64, C.c_uint64, C.c_uint64]),
            "zo_model_create": (C.c_void_p, [C.c_void_p, C.c_int]),
            "zo_model_destroy": (None, [C.c_void_p]),
            "zo_model_prefill_kv_random": (None, [C.c_void_p, C.c_uint32, C.c_uint64]),
            "zo_model_decode_step": (C.c_uint32, [C.c_void_p, C.c_uint32, C.c_uint32, f32p]),
            "zo_model_tensor": (C.c_void_p, [C.c_void_p, C.c_uint64, C.POINTER(C.c_uint64)]),
            "zo_model_tensor_type": (C.c_int, [C.c_void_p, C.c_uint64]),
            "zo_sampling_requires_readback": (C.c_int, [C.c_float, C.c_float, C.c_float]),
            "zo_sample_from_logits": (C.c_uint32, [f32p, C.c_uint32, u32p, C.c_uint32, C.c_float, C.c_float,
                                                   C.c_float, C.c_uint32, C.c_double]),
            "zo_model_set_tensor": (C.c_int, [C.c_void_p, C.c_uint64, C.c_uint32, C.c_void_p, C.c_uint64]),
            "zo_more_bits_layer": (C.c_int, [C.c_uint32, C.c_uint32]),
            "zo_model_hidden": (C.c_void_p, [C.c_void_p]),
            "zo_model_route_gap": (C.c_float, [C.c_void_p]),
            "zo_model_routing": (C.c_int, [C.c_void_p, C.c_uint32, u32p, f32p, C.POINTER(C.c_float)]),
            "zo_model_kv": (C.c_void_p, [C.c_void_p, C.c_uint32, C.c_uint32, C.c_uint32]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def _p(a, ct):
    return a.ctypes.data_as(C.POINTER(ct))


def u8(a):
    return _p(a, C.c_uint8)


def f32(a):
    return _p(a, C.c_float)


def block_size(t):
    return lib().zo_block_size(t)


def bytes_per_block(t):
    return lib().zo_bytes_per_block(t)


def tensor_bytes(t, rows, cols):
    return lib().zo_tensor_bytes(t, rows, cols)


def f16_to_f32(h):
    return lib().zo_f16_to_f32(int(h))


def f32_to_f16(f):
    return lib().zo_f32_to_f16(float(f))


def get_scale_min_k4(j, scales):
    s = np.ascontiguousarray(scales, dtype=np.uint8)
    sc, m = C.c_uint8(), C.c_uint8()
    lib().zo_get_scale_min_k4(j, u8(s), C.byref(sc), C.byref(m))
    return sc.value, m.value


def dequant_row(raw, row, cols, qtype):
    raw = np.ascontiguousarray(raw, dtype=np.uint8)
    out = np.empty(cols, dtype=np.float32)
    rc = lib().zo_dequant_row(u8(raw), row, cols, qtype, f32(out))
    if rc != 0:
        raise ValueError("unsupported quant type %d" % qtype)
    return out


def dequant(raw, rows, cols, qtype):
    return np.stack([dequant_row(raw, r, cols, qtype) for r in range(rows)])


def dmmv(W, qtype, x, M, K, y=None, acc_mode=0, nthreads=8):
    W = np.ascontiguousarray(W, dtype=np.uint8)
    x = np.ascontiguousarray(x, dtype=np.float32)
    if y is None:
        y = np.zeros(M, dtype=np.float32)
    rc = lib().zo_dmmv(u8(W), qtype, f32(x), f32(y), M, K, acc_mode, nthreads)
    if rc != 0:
        raise ValueError("invalid dmmv arguments")
    return y


def dmmv_f64(W, qtype, x, M, K, nthreads=8):
    W = np.ascontiguousarray(W, dtype=np.uint8)
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.zeros(M, dtype=np.float64)
    lib().zo_dmmv_f64(u8(W), qtype, f32(x), _p(y, C.c_double), M, K, nthreads)
    return y


def dmmv_absdot(W, qtype, x, M, K, nthreads=8):
    W = np.ascontiguousarray(W, dtype=np.uint8)
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.zeros(M, dtype=np.float64)
    lib().zo_dmmv_absdot(u8(W), qtype, f32(x), _p(y, C.c_double), M, K, nthreads)
    return y


def rms_norm_mul(x, w, n, n_groups, eps):
    x = np.ascontiguousarray(x, dtype=np.float32)
    w = np.ascontiguousarray(w, dtype=np.float32)
    out = np.empty(n * n_groups, dtype=np.float32)
    lib().zo_rms_norm_mul(f32(x), f32(w), len(w), f32(out), n, n_groups, eps)
    return out


def per_head_rms_norm(x, w, head_dim, n_heads, eps):
    x = np.array(x, dtype=np.float32, copy=True)
    w = np.ascontiguousarray(w, dtype=np.float32)
    lib().zo_per_head_rms_norm(f32(x), f32(w), head_dim, n_heads, eps)
    return x


def rope_inv_freq(rope_dim, base):
    out = np.empty(rope_dim // 2, dtype=np.float32)
    lib().zo_rope_inv_freq(f32(out), rope_dim, base)
    return out


def rope(x, stride, rope_dim, n_heads, position, inv_freq):
    x = np.array(x, dtype=np.float32, copy=True)
    inv = np.ascontiguousarray(inv_freq, dtype=np.float32)
    lib().zo_rope(f32(x), stride, rope_dim, n_heads, position, f32(inv))
    return x


def swiglu(g, u):
    g = np.ascontiguousarray(g, dtype=np.float32)
    u = np.ascontiguousarray(u, dtype=np.float32)
    out = np.empty_like(g)
    lib().zo_swiglu(f32(g), f32(u), f32(out), len(g))
    return out


def attention_f16(q, k16, v16, head_dim, n_heads, n_kv_heads, seq_len, attn_scale=0.0):
    q = np.ascontiguousarray(q, dtype=np.float32)
    k16 = np.ascontiguousarray(k16, dtype=np.uint16)
    v16 = np.ascontiguousarray(v16, dtype=np.uint16)
    out = np.empty(n_heads * head_dim, dtype=np.float32)
    lib().zo_attention_f16(f32(q), _p(k16, C.c_uint16), _p(v16, C.c_uint16), f32(out),
                           head_dim, n_heads, n_kv_heads, seq_len, attn_scale)
    return out


def topk_softmax(logits, k):
    lg = np.ascontiguousarray(logits, dtype=np.float32)
    ids = np.empty(k, dtype=np.uint32)
    w = np.empty(k, dtype=np.float32)
    lib().zo_topk_softmax(f32(lg), len(lg), k, _p(ids, C.c_uint32), f32(w))
    return ids, w


def sample_from_logits(logits, history=(), temperature=0.0, top_p=1.0, repetition_penalty=1.0, top_k=64, u=0.0):
    """sampleFromLogits (forward.zig:10261-10334) with the draw u = random.float(f64)."""
    lg = np.ascontiguousarray(logits, dtype=np.float32)
    h = np.ascontiguousarray(history, dtype=np.uint32)
    if h.size == 0:
        h = np.zeros(1, np.uint32)
        nh = 0
    else:
        nh = h.size
    return int(lib().zo_sample_from_logits(f32(lg), lg.size, _p(h, C.c_uint32), nh, temperature, top_p,
                                           repetition_penalty, top_k, u))


def argmax(logits):
    lg = np.ascontiguousarray(logits, dtype=np.float32)
    return lib().zo_argmax(f32(lg), len(lg))


def rand(seed, stream, ctr):
    return lib().zo_rand(seed, stream, ctr)


def normal(r):
    return lib().zo_normal(r)


def synth_tensor(qtype, rows, cols, seed, stream):
    """qtype | 0x100: centered model-init variant (Q4_K dmin = f16(7.5*d), Q5_K f16(15.5*d))."""
    out = np.empty(tensor_bytes(qtype & 0xFF, rows, cols), dtype=np.uint8)
    if lib().zo_synth_tensor(u8(out), qtype, rows, cols, seed, stream) != 0:
        raise ValueError("bad synth args")
    return out


def synth_normal_f32(n, seed, stream, scale=1.0):
    out = np.empty(n, dtype=np.float32)
    lib().zo_synth_normal_f32(f32(out), n, scale, seed, stream)
    return out


def synth_normal_f16(n, seed, stream):
    out = np.empty(n, dtype=np.uint16)
    lib().zo_synth_normal_f16(_p(out, C.c_uint16), n, seed, stream)
    return out


def synth_norm_weight(n, seed, stream):
    out = np.empty(n, dtype=np.float32)
    lib().zo_synth_norm_weight(f32(out), n, seed, stream)
    return out


class ModelConfig(C.Structure):
    _fields_ = [(n, C.c_uint32) for n in (
        "n_layers", "hidden", "n_heads", "n_kv_heads", "head_dim", "ffn", "vocab",
        "n_experts", "n_experts_used", "expert_ffn", "max_ctx",
        "type_attn", "type_ffn_gate_up", "type_ffn_down", "type_lm_head", "type_embd",
        "type_router")] + [("rope_base", C.c_float), ("eps", C.c_float), ("seed", C.c_uint64),
                            ("type_more_bits", C.c_uint32), ("reserved", C.c_uint32)]


class Model:
    """Whole-model CPU decode (restates decodeStep, forward.zig:4299-7865)."""

    def __init__(self, cfg: dict, nthreads=8):
        self.cfg = dict(cfg)
        c = ModelConfig(**cfg)
        self._c = c
        self.h = lib().zo_model_create(C.byref(c), nthreads)

    def close(self):
        if self.h:
            lib().zo_model_destroy(self.h)
            self.h = None

    def __del__(self):
        self.close()

    def prefill_kv_random(self, n, seed):
        lib().zo_model_prefill_kv_random(self.h, n, seed)

    def decode_step(self, token, pos, want_logits=False):
        logits = np.empty(self.cfg["vocab"], dtype=np.float32) if want_logits else None
        tok = lib().zo_model_decode_step(self.h, token, pos, f32(logits) if want_logits else None)
        return (tok, logits) if want_logits else tok

    def tensor(self, stream):
        n = C.c_uint64()
        p = lib().zo_model_tensor(self.h, stream, C.byref(n))
        if not p:
            return None
        return np.ctypeslib.as_array(C.cast(p, C.POINTER(C.c_uint8)), shape=(n.value,)).copy()

    def tensor_type(self, stream):
        return lib().zo_model_tensor_type(self.h, stream)

    def set_tensor(self, stream, qtype, data):
        """Replace a weight (data: its bytes in storage type qtype)."""
        a = np.ascontiguousarray(np.frombuffer(memoryview(data).cast("B"), dtype=np.uint8))
        rc = lib().zo_model_set_tensor(self.h, stream, qtype, C.c_void_p(a.ctypes.data), a.size)
        if rc != 0:
            raise ValueError(f"zo_model_set_tensor(stream {stream:#x}, type {qtype}, {a.size} B): {rc}")

    def kv(self, layer, which, token):
        """fp16 bits of the K (which=0) or V (1) cache row of `token`."""
        p = lib().zo_model_kv(self.h, layer, which, token)
        n = self.cfg["n_kv_heads"] * self.cfg["head_dim"]
        return np.ctypeslib.as_array(C.cast(p, C.POINTER(C.c_uint16)), shape=(n,)).copy()

    def route_gap(self):
        """Smallest (k-th selected - best unselected) router logit gap of the
        last decode step over its MoE layers, relative to max |router logit|
        (inf for a dense model)."""
        return float(lib().zo_model_route_gap(self.h))

    def routing(self, layer):
        """(selected expert ids, their weights, router gap) of `layer` in the
        last decode step: ids and weights in topKSoftmax's order, the gap as
        route_gap's for that layer alone (inf: no near tie)."""
        k = self.cfg["n_experts_used"]
        ids = np.zeros(16, dtype=np.uint32)
        w = np.zeros(16, dtype=np.float32)
        gap = C.c_float()
        rc = lib().zo_model_routing(self.h, layer, ids.ctypes.data_as(C.POINTER(C.c_uint32)),
                                    w.ctypes.data_as(C.POINTER(C.c_float)), C.byref(gap))
        if rc != 0:
            raise ValueError("routing: dense model or layer out of range")
        return ids[:k].copy(), w[:k].copy(), float(gap.value)

    def hidden(self):
        p = lib().zo_model_hidden(self.h)
        return np.ctypeslib.as_array(C.cast(p, C.POINTER(C.c_float)), shape=(self.cfg["hidden"],)).copy()
