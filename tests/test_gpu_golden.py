"""Full-size parity: the GPU engine decoding the config-3 model (8B-shaped
dense Qwen3, Q4_K_M mix, seeded random-init weights, 4096-token KV prefill)
must reproduce the CPU oracle's 256 greedy tokens exactly. (The opt-in
persistent layers kernel is checked against the oracle model step by step
in test_gpu_engine.py, not through this fixture.) The fixture
tests/golden/dense8b_greedy256.json was written by make_dense8b_golden.py
beside it (the oracle restates forward.zig's decodeStep + sampleGreedy)."""
import json
import os

import pytest

pytestmark = pytest.mark.gpu

FIXTURE = os.path.join(os.path.dirname(__file__), "golden", "dense8b_greedy256.json")


def test_dense8b_greedy_256_token_exact():
    import zinc_amd
    g = json.load(open(FIXTURE))
    cfg = dict(g["config"])
    assert cfg["hidden"] == 4096 and cfg["n_layers"] == 36 and cfg["vocab"] == 151936
    ctx = zinc_amd.Context(0)
    try:
        eng = zinc_amd.InferenceEngine(ctx, cfg)
        eng.prefill_kv_random(g["prefill"], g["kv_seed"])
        got = eng.generate(g["prompt"], len(g["tokens"]), start_pos=g["prefill"])
        eng.deinit()
    finally:
        ctx.close()
    ref = g["tokens"]
    bad = [i for i in range(len(ref)) if got[i] != ref[i]]
    assert not bad, (f"first mismatch at step {bad[0]} (oracle margin there "
                     f"{g['rel_margins'][bad[0]]:.2e} of max |logit|)")


# A greedy step whose top-2 logits the oracle separates by less than this
# fraction of max |logit| is a near tie: a sum in another order may pick the
# other token (the decode tolerance is 1e-3 of the scale). A mismatch there is
# accepted, and the run then continues from the oracle's token (the prompt
# re-decoded with the oracle's tokens appended).
NEAR_TIE = 1e-3
# A routed model adds a second, discrete source of divergence. In a layer
# whose k-th selected router logit beats the best unselected one by a gap
# (relative to the layer's max |router logit|) of the order of the GPU's
# drift from the oracle (the same sums in another order: ~2e-5 of the hidden
# state's scale over 48 layers, up to ~2e-4 of a router logit's), the GPU may
# select the other expert; that moves the step's logits by up to tenths of
# their scale and, through the K/V rows it writes, later steps a little. The
# fixture records each step's smallest gap over its 48 layers. A mismatch is
# accepted at a step whose oracle margin is below NEAR_TIE or whose router gap
# is below ROUTE_FLIP, and at most MAX_ROUTED_MISMATCH steps may mismatch.
# Measured on MI355X (config 4, 256 steps): 2 mismatches, at router gaps of
# 1.4e-5 and 1.3e-4 (the second after the first swapped an expert). The strict
# check is test_moe48_routing_followed_256, which runs the oracle's selection.
ROUTE_FLIP, MAX_ROUTED_MISMATCH = 3e-4, 8


def _greedy_fixture(name):
    import zinc_amd
    g = json.load(open(os.path.join(os.path.dirname(__file__), "golden", name)))
    cfg = dict(g["config"])
    ref, margins = g["tokens"], g["rel_margins"]
    routed = "route_gaps" in g
    gaps = g.get("route_gaps", [1.0] * len(ref))
    print(f"{name}: {cfg['n_layers']} layers, KV prefill {g['prefill']}, {len(ref)} tokens", flush=True)
    ctx = zinc_amd.Context(0)
    ties = []
    try:
        eng = zinc_amd.InferenceEngine(ctx, cfg)
        eng.prefill_kv_random(g["prefill"], g["kv_seed"])
        done = 0
        while done < len(ref):
            got = eng.generate(g["prompt"] + ref[:done], len(ref) - done, start_pos=g["prefill"])
            bad = [i for i in range(len(got)) if got[i] != ref[done + i]]
            if not bad:
                break
            i = done + bad[0]
            print(f"  mismatch at step {i}: oracle margin {margins[i]:.2e}, router gap {gaps[i]:.2e}", flush=True)
            ok = margins[i] < NEAR_TIE or (routed and gaps[i] < ROUTE_FLIP)
            assert ok, (f"mismatch at step {i} (oracle margin there {margins[i]:.2e} of max |logit|, "
                        f"router gap {gaps[i]:.2e})")
            ties.append(i)
            done = i + 1
        eng.deinit()
    finally:
        ctx.close()
    print(f"{name}: token-exact except at near ties {ties}", flush=True)
    assert len(ties) <= (MAX_ROUTED_MISMATCH if routed else len(ref)), ties
    return g


def test_moe48_greedy_256_token_exact():
    """Config 4 at full size: 48 layers, 128 experts top-8 (expert FFN 768,
    experts Q4_K, router and attention Q8_0), LM head Q6_K over 151936, KV
    context 8192, 256 greedy tokens equal to the oracle's except at near ties
    of the logits or the routing (fixture written by
    tests/golden/make_goldens.py moe48)."""
    g = _greedy_fixture("moe48_greedy256.json")
    c = g["config"]
    assert c["n_layers"] == 48 and c["n_experts"] == 128 and c["n_experts_used"] == 8 and c["vocab"] == 151936
    assert g["prefill"] == 8192


# above this router gap the GPU's own selection must be the oracle's: running
# the oracle's experts, its router logits follow the oracle's to ~2e-4 of
# their max (measured: 2 of 12953 compared selections differ, at gaps of
# 2.0e-4 and 1.3e-4)
ROUTE_EXACT = 3e-4


def test_moe48_routing_followed_256():
    """Config 4 at full size, in lockstep with the oracle: every decode step
    (the 15 prompt tokens before the last, then the 256 generated ones) runs
    the oracle's experts in every layer (zh_engine_force_routing) and is fed
    the oracle's token, so no step inherits another expert's K/V rows. Per
    step: the GPU's own selection (what its router top-k computed, recorded
    beside the forced ids) equals the oracle's in every layer whose router gap
    exceeds ROUTE_EXACT (as a set: the order inside the selection is not
    output-relevant), and the greedy token equals the oracle's except at a
    logit near tie (fixtures: moe48_greedy256.json and moe48_routing.npz from
    tests/golden/make_goldens.py moe48)."""
    import numpy as np
    import zinc_amd
    here = os.path.join(os.path.dirname(__file__), "golden")
    g = json.load(open(os.path.join(here, "moe48_greedy256.json")))
    r = np.load(os.path.join(here, "moe48_routing.npz"))
    cfg = dict(g["config"])
    ref, margins = g["tokens"], g["rel_margins"]
    seq = g["prompt"] + ref
    n_pre = len(g["prompt"]) - 1
    assert r["ids"].shape == (n_pre + len(ref), cfg["n_layers"], cfg["n_experts_used"])
    ctx = zinc_amd.Context(0)
    bad_sel, bad_tok, checked = [], [], 0
    try:
        eng = zinc_amd.InferenceEngine(ctx, cfg)
        assert "k_moe_xcd" in eng.group_kernels("ffn")
        eng.prefill_kv_random(g["prefill"], g["kv_seed"])
        st = zinc_amd.DecodeState()
        for s in range(n_pre + len(ref)):
            eng.force_routing(r["ids"][s])
            st.position = g["prefill"] + s
            eng.decode_step(st, seq[s], True)
            for layer in range(cfg["n_layers"]):
                gap = float(r["gaps"][s, layer])
                if gap > ROUTE_EXACT and np.isfinite(gap):
                    checked += 1
                    g_ids, _ = eng.routing(layer)
                    if sorted(g_ids.tolist()) != sorted(r["ids"][s, layer].tolist()):
                        bad_sel.append((s, layer, gap))
            if s >= n_pre:
                i = s - n_pre
                tok = eng.sample_greedy()
                if tok != ref[i]:
                    print(f"  step {i}: token {tok} vs oracle {ref[i]} (oracle margin {margins[i]:.2e})", flush=True)
                    bad_tok.append((i, margins[i]))
        ctx.sync()
        eng.force_routing(None)
        eng.deinit()
    finally:
        ctx.close()
    print(f"moe48 lockstep: {checked} layer selections compared, {len(bad_sel)} differ {bad_sel[:8]}; "
          f"{len(bad_tok)} token mismatches {bad_tok}", flush=True)
    assert not bad_sel, bad_sel[:8]
    assert all(m < NEAR_TIE for _, m in bad_tok), bad_tok


def test_dense8b_32k_greedy_128_token_exact():
    """Config 5's decode: the 8B-shaped model over a 32768-position fp16 KV
    cache (8 kv heads x 128 dims x 36 layers), 128 greedy tokens equal to the
    oracle's (fixture: tests/golden/make_goldens.py dense8b_32k)."""
    g = _greedy_fixture("dense8b_32k_greedy128.json")
    assert g["config"]["n_layers"] == 36 and g["prefill"] == 32768 and len(g["tokens"]) == 128


def test_prefill512_8b_shapes_matches_sequential_oracle():
    """Config 5's prefill: 512 tokens through the MFMA dequant-GEMM path on the
    8B layer shapes (4 layers, vocab 8192) against the oracle decoding the same
    prompt token by token (fixture: tests/golden/make_goldens.py prefill512).
    The GEMMs multiply fp16 operands (the dequantised weights rounded to fp16,
    as the north star's fp16 tiles) with f32 accumulation, so logits and K/V
    rows agree to that rounding, not to the decode path's; the greedy token
    after the prompt and the 15 decoded after it must equal the oracle's."""
    import numpy as np
    import zinc_amd
    f = np.load(os.path.join(os.path.dirname(__file__), "golden", "prefill512_8b4l.npz"))
    cfg = json.loads(str(f["config"]))
    prompt, toks = f["prompt"], f["tokens"].tolist()
    ctx = zinc_amd.Context(0)
    try:
        eng = zinc_amd.InferenceEngine(ctx, cfg)
        eng.prefill(prompt, start_pos=0)
        logits = eng.logits()
        first = eng.sample_greedy()
        kv = np.stack([np.stack([eng.read_kv(cfg["n_layers"] - 1, w, int(r), 1) for r in f["kv_rows"]])
                       for w in (0, 1)])
        cont = eng.generate([first], len(toks) - 1, start_pos=len(prompt))
        eng.deinit()
    finally:
        ctx.close()
    ref = f["logits"].astype(np.float64)
    scale = np.abs(ref).max()
    d = np.abs(logits - ref).max()
    print(f"prefill512: max |logit - oracle| = {d / scale:.2e} of max |logit|", flush=True)
    assert d <= 2e-3 * scale, d / scale
    g32, o32 = kv.view(np.float16).astype(np.float32), f["kv"].view(np.float16).astype(np.float32)
    rowmax = np.abs(o32).max(axis=-1, keepdims=True)
    kd = (np.abs(g32 - o32) / rowmax).max()
    print(f"prefill512: max |K/V - oracle| = {kd:.2e} of the row maximum", flush=True)
    assert kd <= 5e-3, kd
    assert [first] + cont == toks
