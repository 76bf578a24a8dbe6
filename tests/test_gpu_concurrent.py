"""Concurrent sequences: engines sharing one copy of the weights, each on its
own context (HIP stream), decode independent sequences from different host
threads at once. Each sequence's tokens and final logits equal those of the
same engine decoding alone, and one of them equals the oracle's; the
attention merge runs without waiting on other workgroups of its grid
(another stream's kernels may occupy the CUs)."""
import threading

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

SMALL_DENSE = dict(n_layers=3, hidden=512, n_heads=4, n_kv_heads=2, head_dim=128, ffn=1536, vocab=3000,
                   n_experts=0, n_experts_used=0, expert_ffn=0, max_ctx=512,
                   type_attn=12, type_ffn_gate_up=12, type_ffn_down=14, type_lm_head=14, type_embd=12,
                   type_router=8, rope_base=1e6, eps=1e-6, seed=99)


def test_concurrent_sequences_match_alone_and_oracle(orc):
    import zinc_amd
    print("concurrent sequences", flush=True)
    ctxs = [zinc_amd.Context(0) for _ in range(3)]
    base = zinc_amd.InferenceEngine(ctxs[0], SMALL_DENSE)
    engs = [base] + [base.share(c) for c in ctxs[1:]]
    prompts = [[17, 5, 901], [4, 4, 2000, 9], [1234]]
    n_gen = 24

    def run(i, out):
        e = engs[i]
        e.prefill_kv_random(50 + 20 * i, 11 + i)
        out[i] = (e.generate(prompts[i], n_gen, start_pos=50 + 20 * i), e.logits())

    alone = [None] * 3
    for i in range(3):
        run(i, alone)
    together = [None] * 3
    threads = [threading.Thread(target=run, args=(i, together)) for i in range(3)]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=120)
    for i in range(3):
        assert together[i] is not None, f"sequence {i} did not finish"
        assert together[i][0] == alone[i][0], i
        assert np.array_equal(together[i][1], alone[i][1]), i
    # sequence 0 against the oracle's per-token decode
    om = orc.Model(SMALL_DENSE)
    om.prefill_kv_random(50, 11)
    pos, ref = 50, []
    for t in prompts[0][:-1]:
        om.decode_step(t, pos)
        pos += 1
    tok = prompts[0][-1]
    for _ in range(n_gen):
        tok = om.decode_step(tok, pos)
        pos += 1
        ref.append(int(tok))
    assert alone[0][0] == ref
    om.close()
    for e in reversed(engs):
        e.deinit()
    for c in ctxs:
        c.close()
