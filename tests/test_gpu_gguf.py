"""GGUF model files on the GPU engine (loader.load + InferenceEngine.init,
src/model/loader.zig:414-486, forward.zig:1226).

- A model exported to GGUF and loaded back decodes bit-identically to the
  engine it came from (dense and MoE).
- A Q4_K_M-style mix (attn_v / ffn_down in Q6_K on llama.cpp's
  use_more_bits layers, Q4_K elsewhere) decodes like the oracle.
- A file mixing formats per tensor (Q/K/V in three formats, gate and up in
  different ones, ffn_down per layer) feeds both the engine and the oracle
  the same bytes: logits within the decode tolerance, greedy tokens equal.
- Q5_K: a Q5_K_M-style dense mix (Q5_K, Q6_K on the use_more_bits layers,
  Q5_K token embeddings) and a MoE model with Q5_K experts decode like the
  oracle and survive a GGUF round trip.
- Without output.weight the LM head reads token_embd.weight.
- Missing tensors, wrong shapes and formats the kernels do not take fail
  with the reference's errors."""
import numpy as np
import pytest

from zinc_amd import Q4_K, Q5_K, Q6_K, Q8_0, ZincError
from zinc_amd import gguf as G

pytestmark = pytest.mark.gpu

SMALL_DENSE = dict(n_layers=3, hidden=512, n_heads=4, n_kv_heads=2, head_dim=128, ffn=1536, vocab=3000,
                   n_experts=0, n_experts_used=0, expert_ffn=0, max_ctx=512,
                   type_attn=12, type_ffn_gate_up=12, type_ffn_down=14, type_lm_head=14, type_embd=12,
                   type_router=8, rope_base=1e6, eps=1e-6, seed=99)
SMALL_MOE = dict(n_layers=2, hidden=512, n_heads=8, n_kv_heads=1, head_dim=128, ffn=0, vocab=2000,
                 n_experts=16, n_experts_used=4, expert_ffn=256, max_ctx=256,
                 type_attn=8, type_ffn_gate_up=12, type_ffn_down=12, type_lm_head=14, type_embd=12,
                 type_router=8, rope_base=1e6, eps=1e-6, seed=98)
# 8 layers: use_more_bits picks layers 0, 3, 6 and 7
Q4KM_8L = dict(SMALL_DENSE, n_layers=8, type_ffn_down=Q4_K, type_more_bits=Q6_K, seed=95)
Q5KM_8L = dict(SMALL_DENSE, n_layers=8, type_attn=Q5_K, type_ffn_gate_up=Q5_K, type_ffn_down=Q5_K,
               type_embd=Q5_K, type_more_bits=Q6_K, seed=94)
MOE_Q5K = dict(SMALL_MOE, type_ffn_gate_up=Q5_K, type_ffn_down=Q5_K, seed=93)


@pytest.fixture(scope="module")
def ctx():
    import zinc_amd
    c = zinc_amd.Context(0)
    yield c
    c.close()


PROMPT = (17, 5, 901)


def _decode(eng, n_prefill=60, steps=8):
    """One decodeStep's logits and greedy token at position n_prefill, then
    generate() from a fresh KV fill: (step token, step logits, tokens)."""
    import zinc_amd
    eng.prefill_kv_random(n_prefill, 7)
    st = zinc_amd.DecodeState()
    st.position = n_prefill
    eng.decode_step(st, PROMPT[0], True)
    tok, log = eng.sample_greedy(), eng.logits()
    eng.prefill_kv_random(n_prefill, 7)
    return tok, log, eng.generate(list(PROMPT), steps, start_pos=n_prefill)


def _oracle_decode(om, n_prefill=60, steps=8):
    om.prefill_kv_random(n_prefill, 7)
    tok, log = om.decode_step(PROMPT[0], n_prefill, want_logits=True)
    om.prefill_kv_random(n_prefill, 7)
    pos = n_prefill
    for t in PROMPT[:-1]:
        om.decode_step(t, pos)
        pos += 1
    out, t = [], PROMPT[-1]
    for _ in range(steps):
        t = om.decode_step(t, pos)
        pos += 1
        out.append(int(t))
    return tok, log, out


def _close(g, o):
    return np.allclose(g, o, rtol=1e-3, atol=1e-4 + 1e-3 * np.abs(o).max())


@pytest.mark.parametrize("cfg", [SMALL_DENSE, SMALL_MOE], ids=["dense", "moe"])
def test_gguf_roundtrip_bit_identical(ctx, tmp_path, cfg):
    import zinc_amd
    print(f"gguf roundtrip {cfg['n_experts'] and 'moe' or 'dense'}", flush=True)
    src = zinc_amd.InferenceEngine(ctx, cfg)
    path = G.export_engine(src, tmp_path / "m.gguf")
    eng = zinc_amd.InferenceEngine.from_gguf(ctx, path, cfg["max_ctx"])
    for k in ("n_layers", "hidden", "n_heads", "n_kv_heads", "head_dim", "ffn", "vocab", "n_experts",
              "n_experts_used", "expert_ffn", "max_ctx", "type_attn", "type_lm_head", "type_embd"):
        assert eng.config[k] == cfg[k], k
    for stream, name, _ in G.engine_tensor_list(cfg):
        assert eng.tensor_type(stream) == src.tensor_type(stream), name
        assert np.array_equal(eng.tensor_bytes(stream), src.tensor_bytes(stream)), name
    a, b = _decode(src), _decode(eng)
    assert a[0] == b[0] and a[2] == b[2]
    assert np.array_equal(a[1], b[1])
    src.deinit()
    eng.deinit()


def test_q4km_mix_matches_oracle(ctx, orc, tmp_path):
    import zinc_amd
    print("q4km mix vs oracle", flush=True)
    eng = zinc_amd.InferenceEngine(ctx, Q4KM_8L)
    om = orc.Model(Q4KM_8L)
    more = [l for l in range(8) if orc.lib().zo_more_bits_layer(l, 8)]
    assert more == [0, 3, 6, 7]
    for l in range(8):
        want = Q6_K if l in more else Q4_K
        for kind in (orc.K_WV, orc.K_DOWN):
            s = orc.S_LAYER(l, kind)
            assert eng.tensor_type(s) == want and om.tensor_type(s) == want
            assert np.array_equal(eng.tensor_bytes(s), om.tensor(s))
        assert eng.tensor_type(orc.S_LAYER(l, orc.K_WQ)) == Q4_K
    g, o = _decode(eng), _oracle_decode(om)
    assert _close(g[1], o[1]), np.abs(g[1] - o[1]).max()
    assert g[0] == o[0] and g[2] == o[2]
    # and through a GGUF file: identical to the engine it came from
    e2 = zinc_amd.InferenceEngine.from_gguf(ctx, G.export_engine(eng, tmp_path / "q4km.gguf"), Q4KM_8L["max_ctx"])
    g2 = _decode(e2)
    assert g2[0] == g[0] and g2[2] == g[2] and np.array_equal(g2[1], g[1])
    eng.deinit()
    e2.deinit()
    om.close()


@pytest.mark.parametrize("cfg", [Q5KM_8L, MOE_Q5K], ids=["q5km_dense", "moe_q5k_experts"])
def test_q5k_models_match_oracle(ctx, orc, tmp_path, cfg):
    import zinc_amd
    print(f"q5k model vs oracle seed={cfg['seed']}", flush=True)
    eng = zinc_amd.InferenceEngine(ctx, cfg)
    om = orc.Model(cfg)
    kinds = (orc.K_EXP_GATE, orc.K_EXP_UP, orc.K_EXP_DOWN) if cfg["n_experts"] else (orc.K_WQ, orc.K_GATE, orc.K_UP)
    for l in range(cfg["n_layers"]):
        for kind in kinds:
            s = orc.S_LAYER(l, kind)
            assert eng.tensor_type(s) == Q5_K and om.tensor_type(s) == Q5_K
            assert np.array_equal(eng.tensor_bytes(s), om.tensor(s))
    g, o = _decode(eng), _oracle_decode(om)
    assert _close(g[1], o[1]), np.abs(g[1] - o[1]).max()
    assert g[0] == o[0] and g[2] == o[2]
    e2 = zinc_amd.InferenceEngine.from_gguf(ctx, G.export_engine(eng, tmp_path / "q5k.gguf"), cfg["max_ctx"])
    g2 = _decode(e2)
    assert g2[0] == g[0] and g2[2] == g[2] and np.array_equal(g2[1], g[1])
    eng.deinit()
    e2.deinit()
    om.close()


def test_per_tensor_mix_matches_oracle(ctx, orc, tmp_path):
    """Q in Q4_K, K in Q8_0, V in Q6_K (three Q/K/V launches), gate Q4_K with
    up Q6_K (separate mat-vecs + SwiGLU), ffn_down Q4_K / Q6_K / Q8_0 by
    layer, O in Q8_0: the same file into the engine and the oracle."""
    import zinc_amd
    print("per-tensor mix vs oracle", flush=True)
    cfg = SMALL_DENSE
    src = zinc_amd.InferenceEngine(ctx, cfg)
    qd, kvd, H, F = 512, 256, 512, 1536
    shapes = {orc.K_WQ: (qd, H), orc.K_WK: (kvd, H), orc.K_WV: (kvd, H), orc.K_WO: (H, qd),
              orc.K_GATE: (F, H), orc.K_UP: (F, H), orc.K_DOWN: (H, F)}
    mix = {orc.K_WQ: Q4_K, orc.K_WK: Q8_0, orc.K_WV: Q6_K, orc.K_WO: Q8_0, orc.K_GATE: Q4_K, orc.K_UP: Q6_K}
    down = [Q4_K, Q6_K, Q8_0]
    repl = {}
    for l in range(cfg["n_layers"]):
        for kind, t in list(mix.items()) + [(orc.K_DOWN, down[l])]:
            rows, cols = shapes[kind]
            repl[orc.S_LAYER(l, kind)] = (t, orc.synth_tensor(t | 0x100, rows, cols, 4242, orc.S_LAYER(l, kind)))
    tensors = []
    for stream, name, dims in G.engine_tensor_list(cfg):
        t, data = repl.get(stream, (src.tensor_type(stream), None))
        tensors.append((name, dims, t, data if data is not None else src.tensor_bytes(stream)))
    meta = [("general.architecture", "qwen3"), ("qwen3.block_count", (G.U32, 3)),
            ("qwen3.embedding_length", (G.U32, H)), ("qwen3.attention.head_count", (G.U32, 4)),
            ("qwen3.attention.head_count_kv", (G.U32, 2)), ("qwen3.attention.key_length", (G.U32, 128)),
            ("qwen3.feed_forward_length", (G.U32, F)), ("qwen3.rope.freq_base", (G.F32, 1e6)),
            ("qwen3.attention.layer_norm_rms_epsilon", (G.F32, 1e-6))]
    path = tmp_path / "mix.gguf"
    G.write_gguf(path, meta, tensors)
    eng = zinc_amd.InferenceEngine.from_gguf(ctx, path, cfg["max_ctx"])
    om = orc.Model(cfg)
    for stream, (t, data) in repl.items():
        om.set_tensor(stream, t, data)
        assert eng.tensor_type(stream) == t
        assert np.array_equal(eng.tensor_bytes(stream), data)
    g, o = _decode(eng), _oracle_decode(om)
    assert _close(g[1], o[1]), np.abs(g[1] - o[1]).max()
    assert g[0] == o[0] and g[2] == o[2]
    src.deinit()
    eng.deinit()
    om.close()


def test_moe_f32_router_matches_oracle(ctx, orc, tmp_path):
    """llama.cpp keeps ffn_gate_inp (the MoE router) in f32: a qwen3moe file
    with f32 routers loads, and engine and oracle given the same bytes agree."""
    import zinc_amd
    print("moe f32 router vs oracle", flush=True)
    cfg = SMALL_MOE
    src = zinc_amd.InferenceEngine(ctx, cfg)
    rng = np.random.default_rng(17)
    routers = {orc.S_LAYER(l, orc.K_ROUTER): (rng.standard_normal((cfg["n_experts"], cfg["hidden"])) * 0.05)
               .astype(np.float32) for l in range(cfg["n_layers"])}
    tensors = []
    for stream, name, dims in G.engine_tensor_list(cfg):
        if stream in routers:
            tensors.append((name, dims, 0, routers[stream]))
        else:
            tensors.append((name, dims, src.tensor_type(stream), src.tensor_bytes(stream)))
    p = "qwen3moe."
    meta = [("general.architecture", "qwen3moe"), (p + "block_count", (G.U32, cfg["n_layers"])),
            (p + "embedding_length", (G.U32, cfg["hidden"])), (p + "attention.head_count", (G.U32, cfg["n_heads"])),
            (p + "attention.head_count_kv", (G.U32, cfg["n_kv_heads"])), (p + "attention.key_length", (G.U32, 128)),
            (p + "expert_count", (G.U32, cfg["n_experts"])), (p + "expert_used_count", (G.U32, cfg["n_experts_used"])),
            (p + "expert_feed_forward_length", (G.U32, cfg["expert_ffn"])), (p + "rope.freq_base", (G.F32, 1e6)),
            (p + "attention.layer_norm_rms_epsilon", (G.F32, 1e-6))]
    path = tmp_path / "moe_f32router.gguf"
    G.write_gguf(path, meta, tensors)
    eng = zinc_amd.InferenceEngine.from_gguf(ctx, path, cfg["max_ctx"])
    assert eng.config["type_router"] == 0
    om = orc.Model(cfg)
    for stream, w in routers.items():
        om.set_tensor(stream, 0, w)
        assert eng.tensor_type(stream) == 0 and np.array_equal(eng.tensor_bytes(stream).view(np.float32), w.ravel())
    g, o = _decode(eng), _oracle_decode(om)
    assert _close(g[1], o[1]), np.abs(g[1] - o[1]).max()
    assert g[0] == o[0] and g[2] == o[2]
    src.deinit()
    eng.deinit()
    om.close()


def test_tied_embeddings(ctx, tmp_path):
    """No output.weight: the LM head reads token_embd.weight, exactly as a
    file whose output.weight is a copy of token_embd.weight."""
    import zinc_amd
    print("tied embeddings", flush=True)
    src = zinc_amd.InferenceEngine(ctx, SMALL_DENSE)
    tied = zinc_amd.InferenceEngine.from_gguf(ctx, G.export_engine(src, tmp_path / "tied.gguf", tied=True), 512)
    assert tied.config["type_lm_head"] == SMALL_DENSE["type_embd"]
    assert np.array_equal(tied.tensor_bytes(3), src.tensor_bytes(1))
    tensors = [(n, d, src.tensor_type(s), src.tensor_bytes(1 if s == 3 else s))
               for s, n, d in G.engine_tensor_list(SMALL_DENSE)]
    tensors = [(n, d, SMALL_DENSE["type_embd"] if n == "output.weight" else t, b) for n, d, t, b in tensors]
    meta = [(k, v) for k, v in _meta_of(src)]
    G.write_gguf(tmp_path / "copy.gguf", meta, tensors)
    copy = zinc_amd.InferenceEngine.from_gguf(ctx, tmp_path / "copy.gguf", 512)
    a, b = _decode(tied), _decode(copy)
    assert a[0] == b[0] and a[2] == b[2] and np.array_equal(a[1], b[1])
    for e in (src, tied, copy):
        e.deinit()


def _meta_of(eng):
    c = eng.config
    return [("general.architecture", "qwen3"), ("qwen3.block_count", (G.U32, c["n_layers"])),
            ("qwen3.embedding_length", (G.U32, c["hidden"])), ("qwen3.attention.head_count", (G.U32, c["n_heads"])),
            ("qwen3.attention.head_count_kv", (G.U32, c["n_kv_heads"])),
            ("qwen3.attention.key_length", (G.U32, c["head_dim"])),
            ("qwen3.feed_forward_length", (G.U32, c["ffn"])), ("qwen3.rope.freq_base", (G.F32, c["rope_base"])),
            ("qwen3.attention.layer_norm_rms_epsilon", (G.F32, c["eps"]))]


def test_gguf_load_errors(ctx, tmp_path):
    import zinc_amd
    print("gguf load errors", flush=True)
    src = zinc_amd.InferenceEngine(ctx, SMALL_DENSE)
    base = [(n, d, src.tensor_type(s), src.tensor_bytes(s)) for s, n, d in G.engine_tensor_list(SMALL_DENSE)]
    meta = _meta_of(src)

    def load(tensors):
        p = tmp_path / "e.gguf"
        G.write_gguf(p, meta, tensors)
        return zinc_amd.InferenceEngine.from_gguf(ctx, p, 512)

    with pytest.raises(ZincError) as ei:  # a missing layer tensor
        load([t for t in base if t[0] != "blk.1.attn_k.weight"])
    assert ei.value.name == "TensorNotFound"
    bad = [(n, [d[0], d[1] // 2] if n == "blk.0.attn_q.weight" else d, t,
            b[:len(b) // 2] if n == "blk.0.attn_q.weight" else b) for n, d, t, b in base]
    with pytest.raises(ZincError) as ei:  # rows differ from the config
        load(bad)
    assert ei.value.name == "InvalidArgument"
    f16 = [(n, d, 1 if n == "blk.2.ffn_up.weight" else t,
            np.zeros(d[0] * d[1] * 2, np.uint8) if n == "blk.2.ffn_up.weight" else b) for n, d, t, b in base]
    with pytest.raises(ZincError) as ei:  # F16 matrices: no mat-vec kernel here
        load(f16)
    assert ei.value.name == "UnsupportedQuantType"
    # a healthy file still loads after the failures
    e = load(base)
    e.deinit()
    src.deinit()
