"""The output head (output_norm + the Q6_K LM head over the vocabulary +
greedy argmax, forward.zig:7757-7772) at the two hidden sizes of the decode
configs, against the CPU oracle's logits and greedy token: vocabularies
spanning many passes of the workgroups, one smaller than one pass, and odd
ones (which the row-pair kernel does not take: the per-row DMMV runs)."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _cfg(hidden, vocab, seed):
    heads = hidden // 128
    return dict(n_layers=1, hidden=hidden, n_heads=heads, n_kv_heads=heads // 4, head_dim=128, ffn=1024,
                vocab=vocab, n_experts=0, n_experts_used=0, expert_ffn=0, max_ctx=256,
                type_attn=12, type_ffn_gate_up=12, type_ffn_down=14, type_lm_head=14, type_embd=12,
                type_router=8, rope_base=1e6, eps=1e-6, seed=seed)


@pytest.fixture(scope="module")
def ctx():
    import zinc_amd
    c = zinc_amd.Context(0)
    yield c
    c.close()


@pytest.mark.parametrize("hidden,vocab", [(4096, 40000), (4096, 1000), (2048, 40001), (2048, 2999)])
def test_lm_head_matches_oracle(ctx, orc, hidden, vocab):
    import zinc_amd
    cfg = _cfg(hidden, vocab, 60 + vocab % 7)
    eng = zinc_amd.InferenceEngine(ctx, cfg)
    kern = eng.group_kernels("head")
    assert ("LpbP" in kern) == (vocab % 2 == 0), kern
    assert "argmax" in kern
    om = orc.Model(cfg)
    st = zinc_amd.DecodeState()
    for pos, tok in enumerate([5, 17]):
        st.position = pos
        eng.decode_step(st, tok, True)
        g_tok, g_log = eng.sample_greedy(), eng.logits()
        o_tok, o_log = om.decode_step(tok, pos, want_logits=True)
        assert g_log.shape == (vocab,)
        scale = np.abs(o_log).max()
        assert np.abs(g_log - o_log).max() <= 1e-4 + 1e-3 * scale, (pos, np.abs(g_log - o_log).max(), scale)
        assert g_tok == o_tok
    eng.deinit()
