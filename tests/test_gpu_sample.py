"""Device sampling (zh_sample_logits / zh_engine_sample) vs the oracle's
restatement of sampleFromLogits (forward.zig:10261-10334): token-exact for
every parameter set and draw, over logits with NaN, +-inf and tied values,
a repetition-penalty history with repeats and out-of-range ids, and
vocabularies from 3000 to the 262144 maximum."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

PARAMS = [
    dict(),                                                        # greedy (sampleGreedy path)
    dict(temperature=0.0, repetition_penalty=1.3),                 # penalised argmax
    dict(temperature=0.0, top_p=0.5),                              # readback, still greedy
    dict(temperature=0.8, top_k=40),
    dict(temperature=1.2, top_p=0.9, top_k=128),
    dict(temperature=0.5, top_k=1),
    dict(temperature=0.9, top_k=0),                                # clamped to 1
    dict(temperature=0.7, top_k=500),                              # clamped to 128
    dict(temperature=0.7, top_p=0.95, repetition_penalty=1.5, top_k=64),
    dict(temperature=3.0, top_p=0.3, top_k=100),
]
DRAWS = [0.0, 0.1, 0.5, 0.9, 0.999999]


@pytest.fixture(scope="module")
def ctx():
    import zinc_amd
    c = zinc_amd.Context(0)
    yield c
    c.close()


def _logits(n, seed):
    rng = np.random.default_rng(seed)
    lg = rng.normal(0, 3, n).astype(np.float32)
    lg[rng.integers(0, n, 7)] = np.nan
    lg[rng.integers(0, n, 3)] = np.inf
    lg[rng.integers(0, n, 3)] = -np.inf
    top = np.argsort(-np.where(np.isfinite(lg), lg, -1e30))[:200]
    lg[top[60:70]] = lg[top[59]]  # a run of ties inside the candidate range
    return lg


@pytest.mark.parametrize("n", [3000, 151936, 262144])
def test_sample_logits_matches_oracle(ctx, orc, n):
    import zinc_amd
    print(f"sample n={n}", flush=True)
    lg = _logits(n, n)
    rng = np.random.default_rng(5)
    hist = np.concatenate([rng.integers(0, n, 150), rng.integers(0, n, 20).repeat(3), [n + 5, 2**31]])
    hist = hist.astype(np.uint32)
    buf = ctx.upload(lg)
    for p in PARAMS:
        sp = zinc_amd.SamplingParams(**p)
        for u in (DRAWS if sp.draws() else DRAWS[:1]):
            got = ctx.sample_logits(buf, 0, n, sp, hist, u)
            ref = orc.sample_from_logits(lg, hist, sp.temperature, sp.top_p, sp.repetition_penalty, sp.top_k, u)
            assert got == ref, (p, u, got, ref)


def test_sample_greedy_edge_cases(ctx, orc):
    import zinc_amd
    sp = zinc_amd.SamplingParams(temperature=0.0, repetition_penalty=1.2)
    for lg in ([np.nan, 1.0, 2.0], [0.0, np.inf, 1.0], [-np.inf, -np.inf], [np.nan, np.nan], [3.0, 3.0, 1.0]):
        a = np.array(lg, np.float32)
        got = ctx.sample_logits(ctx.upload(a), 0, a.size, sp, [1], 0.4)
        assert got == orc.sample_from_logits(a, [1], 0.0, 1.0, 1.2, 64, 0.4), lg
    # nothing to sample: every logit non-finite
    sp = zinc_amd.SamplingParams(temperature=0.8)
    a = np.array([np.nan, np.inf, -np.inf], np.float32)
    assert ctx.sample_logits(ctx.upload(a), 0, 3, sp, [], 0.7) == 0


def test_sample_distribution(ctx):
    """Over a grid of draws the tokens follow the top-k softmax."""
    import zinc_amd
    rng = np.random.default_rng(11)
    lg = rng.normal(0, 1, 5000).astype(np.float32)
    buf = ctx.upload(lg)
    sp = zinc_amd.SamplingParams(temperature=0.9, top_k=6)
    us = (np.arange(400) + 0.5) / 400
    toks = [ctx.sample_logits(buf, 0, lg.size, sp, [], float(u)) for u in us]
    top = np.argsort(-lg, kind="stable")[:6]
    z = lg[top].astype(np.float64) / 0.9
    p = np.exp(z - z.max())
    p /= p.sum()
    for t, pt in zip(top, p):
        assert abs(toks.count(int(t)) / 400 - pt) < 1 / 400 + 1e-9


def test_engine_sample(ctx, orc):
    import zinc_amd
    cfg = dict(n_layers=2, hidden=512, n_heads=4, n_kv_heads=2, head_dim=128, ffn=1536, vocab=3000,
               n_experts=0, n_experts_used=0, expert_ffn=0, max_ctx=256, type_attn=12, type_ffn_gate_up=12,
               type_ffn_down=14, type_lm_head=14, type_embd=12, type_router=8, rope_base=1e6, eps=1e-6, seed=91)
    eng = zinc_amd.InferenceEngine(ctx, cfg)
    st = zinc_amd.DecodeState()
    st.position = 0
    eng.decode_step(st, 7, True)
    lg = eng.logits()
    st.generated_tokens = [int(np.argmax(lg)), 5, 5, 9]
    draws = iter([0.25, 0.75])
    for p in (dict(), dict(temperature=0.8, top_k=20), dict(temperature=0.0, repetition_penalty=1.4),
              dict(temperature=1.1, top_p=0.8, repetition_penalty=1.2)):
        sp = zinc_amd.SamplingParams(**p)
        u_seen = []

        def rnd():
            u_seen.append(next(draws))
            return u_seen[-1]
        got = eng.sample(st, sp, rnd)
        assert len(u_seen) == (1 if sp.draws() else 0)
        ref = orc.sample_from_logits(lg, st.generated_tokens, sp.temperature, sp.top_p, sp.repetition_penalty,
                                     sp.top_k, u_seen[0] if u_seen else 0.0)
        assert got == ref, p
    eng.deinit()
