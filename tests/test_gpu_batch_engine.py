"""Batched decode (zh_engine_generate_batch): several sequences over one copy
of the weights step in lockstep, the projections as batched DMMV launches.

Each sequence must decode exactly as it does alone (generate() on its own
engine: the single-sequence path that test_gpu_engine.py pins token-exact to
the oracle), and its last logits must agree with that run's within the DMMV
tolerance (the batched path stages the SwiGLU output from f32 where the
single path copies its XQ image, so the last bits may differ)."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

# Q4_K_M-style mix: attn_v / ffn_down Q6_K on the use_more_bits layers, so
# the Q/K/V launches split into runs of equal types; K = 1024 / 2048 keep the
# Q6_K rows 16-byte multiples (the Q6_K tile kernels)
CFG = dict(n_layers=4, hidden=1024, n_heads=8, n_kv_heads=2, head_dim=128, ffn=2048, vocab=4096,
           n_experts=0, n_experts_used=0, expert_ffn=0, max_ctx=512, type_attn=12, type_ffn_gate_up=12,
           type_ffn_down=12, type_lm_head=14, type_embd=12, type_router=8, type_more_bits=14,
           rope_base=1e6, eps=1e-6, seed=57)


@pytest.fixture(scope="module")
def ctx():
    import zinc_amd
    c = zinc_amd.Context(0)
    yield c
    c.close()


@pytest.mark.parametrize("n_seq", [3, 4, 6])
def test_batch_matches_single_sequences(ctx, n_seq):
    import zinc_amd
    print(f"batch engine n_seq={n_seq}", flush=True)
    base = zinc_amd.InferenceEngine(ctx, CFG)
    engines = [base] + [base.share(ctx) for _ in range(n_seq - 1)]
    rng = np.random.default_rng(n_seq)
    prompts = rng.integers(0, CFG["vocab"], (n_seq, 5)).astype(np.uint32)
    prefill, steps = 40, 12
    solo, solo_logits = [], []
    for v, e in enumerate(engines):
        e.prefill_kv_random(prefill, 100 + v)
        solo.append(e.generate(prompts[v].tolist(), steps, start_pos=prefill))
        solo_logits.append(e.logits())
    for v, e in enumerate(engines):
        e.prefill_kv_random(prefill, 100 + v)
    got = zinc_amd.InferenceEngine.generate_batch(engines, prompts, steps, start_pos=prefill)
    for v, e in enumerate(engines):
        assert got[v] == solo[v], (v, got[v], solo[v])
        lg = e.logits()
        ref = solo_logits[v]
        assert np.allclose(lg, ref, rtol=1e-3, atol=1e-4 + 1e-3 * np.abs(ref).max()), (v, np.abs(lg - ref).max())
    assert len({tuple(t) for t in got}) == n_seq  # the sequences really differ
    # a second batched run of the same engine set, after other work on the
    # same stream (a single-sequence decode), repeats the first
    base.prefill_kv_random(prefill, 100)
    assert base.generate(prompts[0].tolist(), steps, start_pos=prefill) == solo[0]
    for v, e in enumerate(engines):
        e.prefill_kv_random(prefill, 100 + v)
    assert zinc_amd.InferenceEngine.generate_batch(engines, prompts, steps, start_pos=prefill) == got
    for e in engines[1:]:
        e.deinit()
    base.deinit()


def test_batch_rejects_foreign_engines(ctx):
    import zinc_amd
    a = zinc_amd.InferenceEngine(ctx, dict(CFG, n_layers=2))
    b = zinc_amd.InferenceEngine(ctx, dict(CFG, n_layers=2, seed=58))  # other weights
    with pytest.raises(zinc_amd.ZincError) as e:
        zinc_amd.InferenceEngine.generate_batch([a, b], [[1, 2], [3, 4]], 2, start_pos=0)
    assert e.value.name == "InvalidArgument"
    with pytest.raises(zinc_amd.ZincError) as e:
        zinc_amd.InferenceEngine.generate_batch([a, a], [[1, 2], [3, 4]], 2, start_pos=0)
    assert e.value.name == "InvalidArgument"
    a.deinit()
    b.deinit()
    # Q8_0 attention: no tile kernel for the batched projections
    q8 = zinc_amd.InferenceEngine(ctx, dict(CFG, n_layers=2, type_attn=8))
    q8b = q8.share(ctx)
    with pytest.raises(zinc_amd.ZincError) as e:
        zinc_amd.InferenceEngine.generate_batch([q8, q8b], [[1, 2], [3, 4]], 2, start_pos=0)
    assert e.value.name == "UnsupportedQuantType"
    q8b.deinit()
    q8.deinit()


def test_batch_groups_on_two_streams(ctx):
    """Two batches of 2 sequences, each on its own context (HIP stream) and
    host thread, decode at once; every sequence as it decodes alone."""
    import threading
    import zinc_amd
    ctx2 = zinc_amd.Context(0)
    cfg = dict(CFG, n_layers=2)
    base = zinc_amd.InferenceEngine(ctx, cfg)
    groups = [[base, base.share(ctx)], [base.share(ctx2), base.share(ctx2)]]
    rng = np.random.default_rng(9)
    prompts = [rng.integers(0, cfg["vocab"], (2, 3)).astype(np.uint32) for _ in range(2)]
    prefill, steps = 30, 10
    solo = []
    for g in range(2):
        for v, e in enumerate(groups[g]):
            e.prefill_kv_random(prefill, 200 + 2 * g + v)
            solo.append(e.generate(prompts[g][v].tolist(), steps, start_pos=prefill))
            e.prefill_kv_random(prefill, 200 + 2 * g + v)
    ctx.sync()
    ctx2.sync()
    got = [None, None]

    def run(g):
        got[g] = zinc_amd.InferenceEngine.generate_batch(groups[g], prompts[g], steps, start_pos=prefill)
    th = [threading.Thread(target=run, args=(g,)) for g in range(2)]
    for t in th:
        t.start()
    for t in th:
        t.join()
    assert got[0] + got[1] == solo
    for e in groups[1] + groups[0][1:]:
        e.deinit()
    base.deinit()
    ctx2.close()
