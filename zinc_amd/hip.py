"""ctypes binding of libzinc_hip.so (include/zinc_hip.h).

This is the Python side of the C ABI: a thin mirror with the same names,
argument meaning and error behaviour (non-zero status -> ZincError carrying
the reference's error name). There is no CPU fallback: if the HIP library is
missing, importing this module's `lib()` raises.
"""
import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.environ.get("ZH_LIB_PATH") or os.path.join(HERE, "libzinc_hip.so")

F32, F16, Q8_0, Q4_K, Q5_K, Q6_K, MXFP4 = 0, 1, 8, 12, 13, 14, 39
OK = 0
STATUS = {1: "UnsupportedQuantType", 2: "InvalidArgument", 3: "HipError",
          4: "ContextLengthExceeded", 5: "OutOfMemory", 6: "TensorNotFound", 7: "InvalidMagic",
          8: "UnknownMetadataType", 9: "UnsupportedArchitecture", 10: "TruncatedFile", 11: "IoError",
          12: "NotFound", 13: "KvCacheExhausted", 14: "WaitTimeout"}

BLOCK = {Q4_K: (256, 144), Q5_K: (256, 176), Q6_K: (256, 210), Q8_0: (32, 34), MXFP4: (32, 17), F32: (1, 4), F16: (1, 2)}


def tensor_bytes(qtype, rows, cols):
    bs, bpb = BLOCK[qtype]
    return rows * (cols // bs) * bpb


class ZincError(RuntimeError):
    def __init__(self, status, msg=""):
        self.status = status
        self.name = STATUS.get(status, "unknown")
        super().__init__(f"{self.name}: {msg}")


class ModelConfig(C.Structure):
    _fields_ = [(n, C.c_uint32) for n in (
        "n_layers", "hidden", "n_heads", "n_kv_heads", "head_dim", "ffn", "vocab",
        "n_experts", "n_experts_used", "expert_ffn", "max_ctx",
        "type_attn", "type_ffn_gate_up", "type_ffn_down", "type_lm_head", "type_embd",
        "type_router")] + [("rope_base", C.c_float), ("eps", C.c_float), ("seed", C.c_uint64),
                            ("type_more_bits", C.c_uint32), ("reserved", C.c_uint32)]


class SamplingParamsC(C.Structure):
    _fields_ = [("temperature", C.c_float), ("top_p", C.c_float), ("repetition_penalty", C.c_float),
                ("top_k", C.c_uint32)]


class SamplingParams:
    """SamplingParams (forward.zig:95-105), with its defaults."""

    def __init__(self, temperature=0.0, top_p=1.0, repetition_penalty=1.0, top_k=64):
        self.temperature, self.top_p = temperature, top_p
        self.repetition_penalty, self.top_k = repetition_penalty, top_k

    def requires_logits_readback(self):
        return self.temperature > 0.0001 or self.top_p < 0.9999 or self.repetition_penalty > 1.0001

    def draws(self):
        """Whether sampleFromLogits draws from the random source (it does so
        only when sampling with a temperature and at least two candidates)."""
        return self.requires_logits_readback() and self.temperature > 0.0001

    def c(self):
        return SamplingParamsC(self.temperature, self.top_p, self.repetition_penalty, self.top_k)


_P = C.c_void_p
_u32, _u64, _f32, _i32 = C.c_uint32, C.c_uint64, C.c_float, C.c_int

SIGNATURES = {
    "zh_init": (_i32, [_i32, C.POINTER(_P)]),
    "zh_destroy": (None, [_P]),
    "zh_last_error": (C.c_char_p, [_P]),
    "zh_status_string": (C.c_char_p, [_i32]),
    "zh_device_info": (_i32, [_P, C.c_char_p, C.c_size_t, C.POINTER(_i32), C.POINTER(_u64)]),
    "zh_sync": (_i32, [_P]),
    "zh_set_attn_wait_limit": (_i32, [_P, _u32]),
    "zh_buf_alloc": (_i32, [_P, _u64, C.POINTER(_P)]),
    "zh_buf_free": (None, [_P, _P]),
    "zh_buf_size": (_u64, [_P]),
    "zh_buf_device_ptr": (_P, [_P]),
    "zh_buf_upload": (_i32, [_P, _P, _u64, _P, _u64]),
    "zh_buf_download": (_i32, [_P, _P, _u64, _P, _u64]),
    "zh_buf_fill_u8": (_i32, [_P, _P, _u64, C.c_uint8, _u64]),
    "zh_event_record": (_i32, [_P, _i32]),
    "zh_event_elapsed_ms": (_i32, [_P, _i32, _i32, C.POINTER(_f32)]),
    "zh_stream_read_probe": (_i32, [_P, _P, _u64, _u32, C.POINTER(_f32)]),
    "zh_synth_tensor": (_i32, [_P, _P, _u64, _u32, _u64, _u64, _u64, _u64]),
    "zh_synth_vector": (_i32, [_P, _P, _u64, _u32, _u64, _f32, _u64, _u64]),
    "zh_dmmv": (_i32, [_P, _u32, _P, _u64, _P, _u64, _P, _u64, _u32, _u32, _u32]),
    "zh_dmmv_fused_gate_up_swiglu": (_i32, [_P, _u32, _P, _u64, _P, _u64, _P, _u64, _P, _u64, _u32, _u32]),
    "zh_dmmv_moe": (_i32, [_P, _u32, _P, _u64, _P, _P, _u32, _u64, _P, _u64, _u32, _u32, _u32]),
    "zh_xq_bytes": (_u64, [_u32]),
    "zh_quantize_activation": (_i32, [_P, _P, _u64, _u32, _u32, _u32, _P, _u64]),
    "zh_dmmv_xq": (_i32, [_P, _u32, _P, _u64, _P, _u64, _P, _u64, _u32, _u32, _u32]),
    "zh_dmmv_batched": (_i32, [_P, _u32, _P, _u64, _P, _u64, _P, _u64, _u32, _u32, _u32, _u32]),
    "zh_dmmv_fused_gate_up_swiglu_batched": (_i32, [_P, _u32, _P, _u64, _P, _u64, _P, _u64, _P, _u64, _u32, _u32,
                                                    _u32]),
    "zh_dmmv_fused_gate_up_swiglu_xq": (_i32, [_P, _u32, _P, _u64, _P, _u64, _P, _u64, _P, _u64, _u32, _u32]),
    "zh_dequant_rows": (_i32, [_P, _u32, _P, _u64, _u32, _u32, _u32, _P, _u64]),
    "zh_rms_norm": (_i32, [_P, _P, _u64, _P, _u32, _P, _u64, _u32, _u32, _f32]),
    "zh_swiglu": (_i32, [_P, _P, _u64, _P, _u64, _P, _u64, _u32]),
    "zh_qk_norm_rope_kv_write": (_i32, [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _u32, _u32, _u32, _u32, _u32,
                                        _u32, _f32]),
    "zh_flash_decode": (_i32, [_P, _P, _P, _P, _P, _u32, _u32, _P, _u32, _u32, _u32, _u32, _f32]),
    "zh_flash_decode_noalloc": (_i32, [_P, _P, _P, _P, _P, _u32, _u32, _P, _u32, _u32, _u32, _u32, _f32]),
    "zh_softmax_topk": (_i32, [_P, _P, _u32, _u32, _P]),
    "zh_moe_weighted_acc": (_i32, [_P, _P, _P, _P, _u32, _u32, _u32]),
    "zh_argmax": (_i32, [_P, _P, _u32, _P, _u64]),
    "zh_engine_prefill": (_i32, [_P, _P, _u32, _u32, _i32]),
    "zh_gemm_xw": (_i32, [_P, _u32, _P, _u64, _P, _u64, _P, _u64, _u32, _u32, _u32, _u32]),
    "zh_engine_create": (_i32, [_P, C.POINTER(ModelConfig), C.POINTER(_P)]),
    "zh_engine_destroy": (None, [_P]),
    "zh_engine_prefill_kv_random": (_i32, [_P, _u32, _u64]),
    "zh_engine_decode_step": (_i32, [_P, _u32, _u32, _i32]),
    "zh_engine_sample_greedy": (_i32, [_P, C.POINTER(_u32)]),
    "zh_engine_generate": (_i32, [_P, _P, _u32, _u32, _u32, _u32, _P, C.POINTER(_u32)]),
    "zh_engine_generate_batch": (_i32, [_P, _u32, _P, _u32, _u32, _u32, _P]),
    "zh_engine_logits": (_i32, [_P, _P]),
    "zh_engine_hidden": (_i32, [_P, _P]),
    "zh_engine_routing": (_i32, [_P, _u32, _P, _P]),
    "zh_engine_force_routing": (_i32, [_P, _P, _u32]),
    "zh_engine_tensor": (_i32, [_P, _u64, C.POINTER(_P), C.POINTER(_u64), C.POINTER(_u64)]),
    "zh_engine_read_kv": (_i32, [_P, _u32, _u32, _u32, _u32, _P]),
    "zh_engine_set_pages": (_i32, [_P, _P, _u32]),
    "zh_engine_set_persistent": (_i32, [_P, _i32]),
    "zh_engine_set_fused_attn": (_i32, [_P, _i32]),
    "zh_engine_set_fused_ffn": (_i32, [_P, _i32]),
    "zh_dmmv_supported": (_i32, [_u32, _u32]),
    "zh_engine_group_kernels": (_i32, [_P, _u32, C.c_char_p, C.c_size_t]),
    "zh_kv_pool_create": (_i32, [_u32, _u32, C.POINTER(_P)]),
    "zh_kv_pool_destroy": (None, [_P]),
    "zh_kv_pool_alloc": (_i32, [_P, _u64, _u32, _P]),
    "zh_kv_pool_free": (None, [_P, _u64]),
    "zh_kv_pool_free_count": (_u32, [_P]),
    "zh_kv_pool_max_context": (_u32, [_P, _u32]),
    "zh_engine_bytes_per_token": (_u64, [_P, _u32]),
    "zh_engine_time_kernel": (_i32, [_P, _u32, _u32, _P]),
    "zh_engine_group_bytes": (_u64, [_P, _u32, _u32]),
    "zh_engine_tensor_type": (_i32, [_P, _u64, C.POINTER(_u32)]),
    "zh_flash_attn_batched": (_i32, [_P, _P, _P, _P, _P, _u32, _u32, _P, _u32, _u32, _u32, _u32, _u32, _f32]),
    "zh_sample_logits": (_i32, [_P, _P, _u64, _u32, C.POINTER(SamplingParamsC), _P, _u32, C.c_double,
                                C.POINTER(_u32)]),
    "zh_engine_sample": (_i32, [_P, C.POINTER(SamplingParamsC), _P, _u32, C.c_double, C.POINTER(_u32)]),
    "zh_engine_create_gguf": (_i32, [_P, _P, _u32, C.POINTER(_P)]),
    "zh_engine_create_shared": (_i32, [_P, _P, _u32, C.POINTER(_P)]),
    "zh_gguf_open": (_i32, [C.c_char_p, C.POINTER(_P)]),
    "zh_gguf_close": (None, [_P]),
    "zh_gguf_last_error": (C.c_char_p, [_P]),
    "zh_gguf_version": (_u32, [_P]),
    "zh_gguf_tensor_count": (_u64, [_P]),
    "zh_gguf_metadata_count": (_u64, [_P]),
    "zh_gguf_data_offset": (_u64, [_P]),
    "zh_gguf_data": (_P, [_P]),
    "zh_gguf_file_size": (_u64, [_P]),
    "zh_gguf_tensor_info": (_i32, [_P, _u64, C.POINTER(C.c_char_p), C.POINTER(_u32), C.POINTER(_u64),
                                   C.POINTER(_u32), C.POINTER(_u64), C.POINTER(_u64)]),
    "zh_gguf_find_tensor": (C.c_int64, [_P, C.c_char_p]),
    "zh_gguf_get_u32": (_i32, [_P, C.c_char_p, C.POINTER(_u32)]),
    "zh_gguf_get_u64": (_i32, [_P, C.c_char_p, C.POINTER(_u64)]),
    "zh_gguf_get_f32": (_i32, [_P, C.c_char_p, C.POINTER(_f32)]),
    "zh_gguf_get_bool": (_i32, [_P, C.c_char_p, C.POINTER(_i32)]),
    "zh_gguf_get_string": (_i32, [_P, C.c_char_p, C.POINTER(C.c_char_p), C.POINTER(_u64)]),
    "zh_gguf_metadata_entry": (_i32, [_P, _u64, C.POINTER(C.c_char_p), C.POINTER(_u32), C.POINTER(_u32),
                                      C.POINTER(_u64)]),
    "zh_gguf_model_config": (_i32, [_P, _u32, _P]),
}

_lib = None


def lib():
    """Load libzinc_hip.so. Raises (never falls back) when it is missing."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is not built: run `python -m zinc_amd.build`")
        L = C.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def _ptr(a):
    return C.c_void_p(a.ctypes.data)


class Buffer:
    """Device buffer (zh_buf): owned by its Context."""

    def __init__(self, ctx, size):
        self.ctx = ctx
        h = C.c_void_p()
        ctx.check(lib().zh_buf_alloc(ctx.h, size, C.byref(h)))
        self.h = h
        self.size = size

    def free(self):
        if self.h:
            lib().zh_buf_free(self.ctx.h, self.h)
            self.h = None

    def upload(self, arr, offset=0):
        a = np.ascontiguousarray(arr)
        self.ctx.check(lib().zh_buf_upload(self.ctx.h, self.h, offset, _ptr(a), a.nbytes))
        return self

    def download(self, dtype, count, offset=0):
        out = np.empty(count, dtype=dtype)
        self.ctx.check(lib().zh_buf_download(self.ctx.h, self.h, offset, _ptr(out), out.nbytes))
        return out

    @property
    def device_ptr(self):
        return lib().zh_buf_device_ptr(self.h)


class Context:
    """zh_ctx: one device + one HIP stream."""

    def __init__(self, device=0):
        h = C.c_void_p()
        rc = lib().zh_init(device, C.byref(h))
        if rc != OK:
            raise ZincError(rc, f"zh_init({device})")
        self.h = h
        self._bufs = []

    def check(self, rc):
        if rc != OK:
            raise ZincError(rc, lib().zh_last_error(self.h).decode())
        return rc

    def close(self):
        if self.h:
            for b in self._bufs:
                b.free()
            self._bufs = []
            lib().zh_destroy(self.h)
            self.h = None

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    def info(self):
        name = C.create_string_buffer(256)
        cu, hbm = C.c_int(), C.c_uint64()
        self.check(lib().zh_device_info(self.h, name, 256, C.byref(cu), C.byref(hbm)))
        return name.value.decode(), cu.value, hbm.value

    def sync(self):
        self.check(lib().zh_sync(self.h))

    def set_attn_wait_limit(self, microseconds):
        """Bound of the decode attention's merge wait (0: give up at once)."""
        self.check(lib().zh_set_attn_wait_limit(self.h, int(microseconds)))

    def alloc(self, size):
        b = Buffer(self, size)
        self._bufs.append(b)
        return b

    def free(self, b):
        if b in self._bufs:
            self._bufs.remove(b)
        b.free()

    def upload(self, arr):
        a = np.ascontiguousarray(arr)
        return self.alloc(max(a.nbytes, 4)).upload(a)

    def record(self, slot):
        self.check(lib().zh_event_record(self.h, slot))

    def elapsed_ms(self, a, b):
        ms = C.c_float()
        self.check(lib().zh_event_elapsed_ms(self.h, a, b, C.byref(ms)))
        return ms.value

    def stream_read_probe(self, buf, nbytes, iters=20):
        g = C.c_float()
        self.check(lib().zh_stream_read_probe(self.h, buf.h, nbytes, iters, C.byref(g)))
        return g.value

    # ---- ops (thin wrappers; argument meaning as include/zinc_hip.h) ----
    def synth_tensor(self, buf, offset, qtype, rows, cols, seed, stream):
        self.check(lib().zh_synth_tensor(self.h, buf.h, offset, qtype, rows, cols, seed, stream))

    def synth_vector(self, buf, offset, kind, n, scale, seed, stream):
        self.check(lib().zh_synth_vector(self.h, buf.h, offset, kind, n, scale, seed, stream))

    def dmmv(self, qtype, W, a_off, x, x_off, y, y_off, M, K, acc_mode=0):
        self.check(lib().zh_dmmv(self.h, qtype, W.h, a_off, x.h, x_off, y.h, y_off, M, K, acc_mode))

    def dmmv_fused_gate_up_swiglu(self, qtype, Wg, g_off, Wu, u_off, x, x_off, y, y_off, M, K):
        self.check(lib().zh_dmmv_fused_gate_up_swiglu(self.h, qtype, Wg.h, g_off, Wu.h, u_off, x.h, x_off,
                                                      y.h, y_off, M, K))

    def dmmv_batched(self, qtype, W, a_off, X, x_off, Y, y_off, M, K, num_cols, acc_mode=0):
        """recordBatchDispatchPush: Y[v] (+)= W X[v], X [num_cols][K], Y [num_cols][M]."""
        self.check(lib().zh_dmmv_batched(self.h, qtype, W.h, a_off, X.h, x_off, Y.h, y_off, M, K, num_cols,
                                          acc_mode))

    def dmmv_fused_gate_up_swiglu_batched(self, qtype, Wg, g_off, Wu, u_off, X, x_off, Y, y_off, M, K, num_cols):
        self.check(lib().zh_dmmv_fused_gate_up_swiglu_batched(self.h, qtype, Wg.h, g_off, Wu.h, u_off, X.h, x_off,
                                                              Y.h, y_off, M, K, num_cols))

    def dmmv_moe(self, qtype, W, expert_stride, routing, x, x_expert_stride, x_off, y, y_off, M, K, n_used):
        self.check(lib().zh_dmmv_moe(self.h, qtype, W.h, expert_stride, routing.h, x.h, x_expert_stride, x_off,
                                     y.h, y_off, M, K, n_used))

    def xq_bytes(self, K):
        return lib().zh_xq_bytes(K)

    def quantize_activation(self, x, x_off, K, xq, xq_off=0, n_vec=1, x_stride=0):
        self.check(lib().zh_quantize_activation(self.h, x.h, x_off, K, n_vec, x_stride, xq.h, xq_off))

    def dmmv_xq(self, qtype, W, a_off, xq, xq_off, y, y_off, M, K, acc_mode=0):
        self.check(lib().zh_dmmv_xq(self.h, qtype, W.h, a_off, xq.h, xq_off, y.h, y_off, M, K, acc_mode))

    def dmmv_fused_gate_up_swiglu_xq(self, qtype, Wg, g_off, Wu, u_off, xq, xq_off, y, y_off, M, K):
        self.check(lib().zh_dmmv_fused_gate_up_swiglu_xq(self.h, qtype, Wg.h, g_off, Wu.h, u_off, xq.h, xq_off,
                                                         y.h, y_off, M, K))

    def dequant_rows(self, qtype, W, a_off, row0, n_rows, K, out, out_off=0):
        self.check(lib().zh_dequant_rows(self.h, qtype, W.h, a_off, row0, n_rows, K, out.h, out_off))

    def rms_norm(self, x, x_off, w, w_len, out, out_off, n, n_groups, eps):
        self.check(lib().zh_rms_norm(self.h, x.h, x_off, w.h, w_len, out.h, out_off, n, n_groups, eps))

    def swiglu(self, g, u, out, n):
        self.check(lib().zh_swiglu(self.h, g.h, 0, u.h, 0, out.h, 0, n))

    def qk_norm_rope_kv_write(self, q, qw, k, kw, v, inv_freq, kc, vc, pages, n_pages, cache_tokens,
                              nq, nkv, hd, position, eps):
        self.check(lib().zh_qk_norm_rope_kv_write(self.h, q.h, qw.h, k.h, kw.h, v.h, inv_freq.h, kc.h, vc.h,
                                                  pages.h, n_pages, cache_tokens, nq, nkv, hd, position, eps))

    def flash_decode(self, q, kc, vc, pages, n_pages, cache_tokens, out, nh, nkv, hd, seq_len, attn_scale=0.0):
        self.check(lib().zh_flash_decode(self.h, q.h, kc.h, vc.h, pages.h, n_pages, cache_tokens, out.h, nh,
                                         nkv, hd, seq_len, attn_scale))

    def flash_decode_noalloc(self, q, kc, vc, pages, n_pages, cache_tokens, out, nh, nkv, hd, seq_len,
                             attn_scale=0.0):
        self.check(lib().zh_flash_decode_noalloc(self.h, q.h, kc.h, vc.h, pages.h, n_pages, cache_tokens, out.h,
                                                 nh, nkv, hd, seq_len, attn_scale))

    def softmax_topk(self, logits, n, k, routing):
        self.check(lib().zh_softmax_topk(self.h, logits.h, n, k, routing.h))

    def moe_weighted_acc(self, a, b, routing, n, n_used, src_stride):
        self.check(lib().zh_moe_weighted_acc(self.h, a.h, b.h, routing.h, n, n_used, src_stride))

    def argmax(self, logits, n, result, result_off=0):
        self.check(lib().zh_argmax(self.h, logits.h, n, result.h, result_off))

    def flash_attn_batched(self, q, kc, vc, pages, n_pages, cache_tokens, out, nh, nkv, hd, seq_start, n, scale=0.0):
        self.check(lib().zh_flash_attn_batched(self.h, q.h, kc.h, vc.h, pages.h, n_pages, cache_tokens, out.h, nh, nkv,
                                               hd, seq_start, n, scale))

    def sample_logits(self, logits, off, n, params, history=(), u=0.0):
        """sampleFromLogits on the device (u: the random.float(f64) draw)."""
        h = np.ascontiguousarray(history, dtype=np.uint32)
        t = C.c_uint32()
        pc = params.c()
        self.check(lib().zh_sample_logits(self.h, logits.h, off, n, C.byref(pc), _ptr(h) if h.size else None,
                                          h.size, u, C.byref(t)))
        return t.value

    def gemm_xw(self, qtype, W, a_off, X, x_off, Y, y_off, M, K, N, acc_mode=0):
        """Y[n][m] (+)= X[n] . W[m] for N tokens (X fp16 [N][K], Y f32 [N][M])."""
        self.check(lib().zh_gemm_xw(self.h, qtype, W.h, a_off, X.h, x_off, Y.h, y_off, M, K, N, acc_mode))
