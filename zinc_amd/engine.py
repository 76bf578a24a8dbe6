"""Python mirror of the reference engine surface (src/compute/forward.zig):
InferenceEngine.init / decodeStep / sampleGreedy / deinit and the free
function generate, over the HIP engine in libzinc_hip.so."""
import ctypes as C

import numpy as np

from . import hip
from .hip import Q4_K, Q6_K, Q8_0, ModelConfig, lib

# 8B-shaped dense decoder, Q4_K_M mix (Q4_K attention/FFN,
# Q6_K ffn_down and lm-head).
DENSE_8B = dict(n_layers=36, hidden=4096, n_heads=32, n_kv_heads=8, head_dim=128, ffn=12288, vocab=151936,
                n_experts=0, n_experts_used=0, expert_ffn=0, max_ctx=4096 + 16 + 256,
                type_attn=Q4_K, type_ffn_gate_up=Q4_K, type_ffn_down=Q6_K, type_lm_head=Q6_K, type_embd=Q4_K,
                type_router=Q8_0, rope_base=1e6, eps=1e-6, seed=1237)

# sparse MoE, 48 layers, 128 experts top-8, expert FFN 768;
# experts Q4_K, router/attention Q8_0, lm-head Q6_K.
MOE_48L = dict(n_layers=48, hidden=2048, n_heads=32, n_kv_heads=4, head_dim=128, ffn=0, vocab=151936,
               n_experts=128, n_experts_used=8, expert_ffn=768, max_ctx=8192 + 16 + 256,
               type_attn=Q8_0, type_ffn_gate_up=Q4_K, type_ffn_down=Q4_K, type_lm_head=Q6_K, type_embd=Q4_K,
               type_router=Q8_0, rope_base=1e6, eps=1e-6, seed=1238)


class DecodeState:
    """DecodeState (forward.zig:63-92)."""

    def __init__(self):
        self.position = 0
        self.generated_tokens = []
        self.requested_context_tokens = 0


class InferenceEngine:
    def __init__(self, ctx: hip.Context, config: dict):
        self.ctx = ctx
        self.config = dict(config)
        self._cfg = ModelConfig(**self.config)
        h = C.c_void_p()
        ctx.check(lib().zh_engine_create(ctx.h, C.byref(self._cfg), C.byref(h)))
        self.h = h

    @classmethod
    def from_gguf(cls, ctx: hip.Context, path, max_ctx=0):
        """loader.load + InferenceEngine.init (loader.zig:414-486,
        forward.zig:1226): an engine on a GGUF file's weights, each tensor in
        its stored format. max_ctx: KV capacity in tokens (0: the file's
        context_length)."""
        from .gguf import GGUFFile
        with GGUFFile(path) as f:
            eng = cls.__new__(cls)
            eng.ctx = ctx
            eng.config = f.model_config(max_ctx)
            eng._cfg = ModelConfig(**eng.config)
            h = C.c_void_p()
            ctx.check(lib().zh_engine_create_gguf(ctx.h, f.h, max_ctx, C.byref(h)))
            eng.h = h
        return eng

    def share(self, ctx: hip.Context, max_ctx=0):
        """A second engine over these weights on `ctx` (its own stream, KV
        cache and activations), for decoding another sequence concurrently
        from another host thread. Deinit it before this engine."""
        eng = type(self).__new__(type(self))
        eng.ctx = ctx
        eng.config = dict(self.config)
        if max_ctx:
            eng.config["max_ctx"] = (max_ctx + 15) // 16 * 16
        eng._cfg = ModelConfig(**eng.config)
        h = C.c_void_p()
        ctx.check(lib().zh_engine_create_shared(ctx.h, self.h, max_ctx, C.byref(h)))
        eng.h = h
        return eng

    def deinit(self):
        if self.h:
            lib().zh_engine_destroy(self.h)
            self.h = None

    close = deinit

    def prefill_kv_random(self, n_tokens, seed):
        self.ctx.check(lib().zh_engine_prefill_kv_random(self.h, n_tokens, seed))

    def decode_step(self, state: DecodeState, token_id: int, collect_output: bool = True):
        """decodeStep (forward.zig:4299): one token at state.position."""
        self.ctx.check(lib().zh_engine_decode_step(self.h, token_id, state.position, int(collect_output)))
        state.position += 1

    def prefill(self, tokens, start_pos=0, collect_output=True, state: DecodeState = None):
        """prefillBatched (forward.zig:9330): all tokens at once (MFMA GEMMs);
        state.position (if given) advances past them."""
        p = np.ascontiguousarray(tokens, dtype=np.uint32)
        self.ctx.check(lib().zh_engine_prefill(self.h, C.c_void_p(p.ctypes.data), len(p), start_pos,
                                               int(collect_output)))
        if state is not None:
            state.position = start_pos + len(p)

    def sample_greedy(self) -> int:
        t = C.c_uint32()
        self.ctx.check(lib().zh_engine_sample_greedy(self.h, C.byref(t)))
        return t.value

    def sample(self, state: DecodeState, params, random=None):
        """InferenceEngine.sample (forward.zig:10360-10367): sampleGreedy when
        the params need no logits, else sampleFromLogits on the device over
        the last step's logits with state.generated_tokens as the history.
        random: a callable returning a float in [0, 1) (the reference's
        random.float(f64)); called only when the params sample."""
        h = np.ascontiguousarray(state.generated_tokens, dtype=np.uint32)
        u = float(random()) if params.draws() else 0.0
        t = C.c_uint32()
        pc = params.c()
        self.ctx.check(lib().zh_engine_sample(self.h, C.byref(pc), C.c_void_p(h.ctypes.data) if h.size else None,
                                              h.size, u, C.byref(t)))
        return t.value

    def generate(self, prompt, max_tokens, eos=0xFFFFFFFF, start_pos=0):
        """generate (forward.zig:10983): prompt then greedy decode on device."""
        p = np.ascontiguousarray(prompt, dtype=np.uint32)
        out = np.zeros(max(max_tokens, 1), dtype=np.uint32)
        n = C.c_uint32()
        self.ctx.check(lib().zh_engine_generate(self.h, C.c_void_p(p.ctypes.data), len(p), start_pos, max_tokens,
                                                eos, C.c_void_p(out.ctypes.data), C.byref(n)))
        return out[:n.value].tolist()

    @staticmethod
    def generate_batch(engines, prompts, max_tokens, start_pos=0):
        """Greedy decode of len(engines) sequences in lockstep on one weight
        stream (zh_engine_generate_batch): engines[0] and engines built with
        share() on its context; prompts: one equal-length prompt per engine.
        Returns one token list per sequence."""
        n = len(engines)
        P = np.ascontiguousarray(prompts, dtype=np.uint32)
        if P.ndim != 2 or P.shape[0] != n:
            raise ValueError("one prompt per engine, all of the same length")
        out = np.zeros((n, max(max_tokens, 1)), dtype=np.uint32)
        hs = (C.c_void_p * n)(*[e.h for e in engines])
        engines[0].ctx.check(lib().zh_engine_generate_batch(hs, n, C.c_void_p(P.ctypes.data), P.shape[1], start_pos,
                                                            max_tokens, C.c_void_p(out.ctypes.data)))
        return [out[v, :max_tokens].tolist() for v in range(n)]

    def logits(self):
        out = np.empty(self.config["vocab"], dtype=np.float32)
        self.ctx.check(lib().zh_engine_logits(self.h, C.c_void_p(out.ctypes.data)))
        return out

    def hidden(self):
        out = np.empty(self.config["hidden"], dtype=np.float32)
        self.ctx.check(lib().zh_engine_hidden(self.h, C.c_void_p(out.ctypes.data)))
        return out

    def routing(self, layer):
        """(expert ids, routing weights) the last step selected in `layer`."""
        k = self.config["n_experts_used"]
        ids, w = np.empty(k, dtype=np.uint32), np.empty(k, dtype=np.float32)
        self.ctx.check(lib().zh_engine_routing(self.h, layer, C.c_void_p(ids.ctypes.data), C.c_void_p(w.ctypes.data)))
        return ids, w

    def force_routing(self, ids):
        """Run the given experts ([n_layers][n_experts_used]) instead of the
        MoE launch's own selection (None: off); test hook."""
        if ids is None:
            self.ctx.check(lib().zh_engine_force_routing(self.h, None, 0))
            return
        a = np.ascontiguousarray(ids, dtype=np.uint32)
        self.ctx.check(lib().zh_engine_force_routing(self.h, C.c_void_p(a.ctypes.data), a.size))

    def tensor_bytes(self, stream):
        b, off, n = C.c_void_p(), C.c_uint64(), C.c_uint64()
        self.ctx.check(lib().zh_engine_tensor(self.h, stream, C.byref(b), C.byref(off), C.byref(n)))
        out = np.empty(n.value, dtype=np.uint8)
        self.ctx.check(lib().zh_buf_download(self.ctx.h, b, off.value, C.c_void_p(out.ctypes.data), n.value))
        return out

    def tensor_type(self, stream):
        t = C.c_uint32()
        self.ctx.check(lib().zh_engine_tensor_type(self.h, stream, C.byref(t)))
        return t.value

    def read_kv(self, layer, which, t0, n):
        c = self.config
        out = np.empty(n * c["n_kv_heads"] * c["head_dim"], dtype=np.uint16)
        self.ctx.check(lib().zh_engine_read_kv(self.h, layer, which, t0, n, C.c_void_p(out.ctypes.data)))
        return out

    def set_pages(self, pages):
        """The sequence's KV page table (logical page i -> physical pages[i])."""
        a = np.ascontiguousarray(pages, dtype=np.uint32)
        self.ctx.check(lib().zh_engine_set_pages(self.h, C.c_void_p(a.ctypes.data), len(a)))

    def set_persistent(self, on=True):
        """Run the step's layers as one persistent launch where the model takes it."""
        self.ctx.check(lib().zh_engine_set_persistent(self.h, int(bool(on))))

    def set_fused_attn(self, on=True):
        """Q/K/V projection and attention in one launch where the model takes it (default on)."""
        self.ctx.check(lib().zh_engine_set_fused_attn(self.h, int(bool(on))))

    def set_fused_ffn(self, on=True):
        """The dense FFN as one per-XCD launch where the model takes it (default on)."""
        self.ctx.check(lib().zh_engine_set_fused_ffn(self.h, int(bool(on))))

    def bytes_per_token(self, L):
        return lib().zh_engine_bytes_per_token(self.h, L)

    # per-layer launch groups of the decode step (zinc_hip.h ZH_GROUP_*)
    GROUPS = {"qkv": 1, "attn": 2, "qkv_attn": 3, "qkv_attn_o": 7, "o": 4, "ffn_in": 8, "ffn_out": 16, "ffn": 24,
              "head": 32}

    def time_kernel(self, group, iters=200):
        """Average us per launch of one launch group, replayed with the
        engine's own arguments rotating through the layers."""
        us = C.c_float()
        self.ctx.check(lib().zh_engine_time_kernel(self.h, self.GROUPS[group], iters, C.byref(us)))
        return us.value

    def head_us(self, iters=20):
        """Output norm + LM head + argmax, us per launch group."""
        return self.time_kernel("head", iters)

    def group_kernels(self, group):
        """Names of the kernels one launch group launches (as captured)."""
        buf = C.create_string_buffer(4096)
        self.ctx.check(lib().zh_engine_group_kernels(self.h, self.GROUPS[group], buf, 4096))
        return buf.value.decode()

    def group_bytes(self, group, L):
        return lib().zh_engine_group_bytes(self.h, self.GROUPS[group], L)


class KvPagePool:
    """KvPagePool (src/scheduler/kv_cache.zig:43-125) over zh_kv_pool_*:
    alloc_pages pops page ids off a free stack (a fresh pool hands them out
    in descending order) and raises ZincError("KvCacheExhausted") when too few
    are free; free_pages returns every page a request owns."""

    def __init__(self, total_pages, page_size=16):
        h = C.c_void_p()
        rc = lib().zh_kv_pool_create(total_pages, page_size, C.byref(h))
        if rc != hip.OK:
            raise hip.ZincError(rc, "zh_kv_pool_create")
        self.h = h
        self.page_size = page_size

    def alloc_pages(self, request_id, count):
        out = np.empty(count, dtype=np.uint32)
        rc = lib().zh_kv_pool_alloc(self.h, request_id, count, C.c_void_p(out.ctypes.data))
        if rc != hip.OK:
            raise hip.ZincError(rc, f"alloc {count} pages")
        return out

    def free_pages(self, request_id):
        lib().zh_kv_pool_free(self.h, request_id)

    def free_count(self):
        return lib().zh_kv_pool_free_count(self.h)

    def max_context(self, page_count):
        return lib().zh_kv_pool_max_context(self.h, page_count)

    def close(self):
        if self.h:
            lib().zh_kv_pool_destroy(self.h)
            self.h = None

    def __del__(self):
        self.close()
