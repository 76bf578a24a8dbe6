"""Per-kernel roofline of the 8B-shape decode step, and the launch sequence
its hardware-counter profile is taken from.

Every per-layer launch group of the decode step (Q/K/V with attn_norm fused,
attention, O projection, gate/up + SwiGLU with ffn_norm fused, down
projection) is replayed by the engine itself (zh_engine_time_kernel) with its
own arguments and state, rotating through the 36 layers so the weights stream
from HBM (4.9 GB of weights > 256 MB MALL). Each group is one kernel in the
dense model; achieved GB/s = the group's algorithmic bytes per launch
(zh_engine_group_bytes: weights, activation in/out, KV rows) / the average
launch duration by HIP events on the engine's stream. The dominant kernel is
the group with the largest duration (each runs once per layer, so also the
largest share of step time).

    python -m benchmarks.roofline_probe            # per-kernel table (JSON)
    rocprofv3 --pmc FETCH_SIZE -- python3 -m benchmarks.roofline_probe --pmc
    rocprofv3 --pmc FETCH_SIZE -- python3 -m benchmarks.roofline_probe --pmc --config 4

--config 4 takes config 4's model instead (48-layer sparse MoE, hidden
2048, KV context 8192): its two per-layer launches, the attention launch and
the MoE FFN launch (whose algorithmic bytes count the 8 experts each layer
selects in the replayed state).

With --pmc the script launches, in order: a streaming read of CAL_BYTES
(known size), a write of CAL_BYTES (known size), then for each group in
GROUP_ORDER one warm pass over the layers and PMC_ITERS timed launches;
benchmarks.pmc_summary turns the counters into bytes per launch.
"""
import argparse
import json
import sys

from zinc_amd import hip
from zinc_amd.engine import DENSE_8B, MOE_48L, InferenceEngine

PEAK = 8000.0
CAL_BYTES = 1 << 30      # calibration read / write size
PREFILL = 4096           # KV context of the bench (config 3)
PREFILL_C4 = 8192        # KV context of config 4
GROUP_ORDER = ["qkv", "attn", "o", "ffn_in", "ffn_out"]
PMC_ITERS = 36


def probe_engine(ctx, max_ctx, model=DENSE_8B, prefill=PREFILL):
    cfg = dict(model)
    cfg["max_ctx"] = max_ctx
    eng = InferenceEngine(ctx, cfg)
    eng.prefill_kv_random(prefill, 7)
    eng.generate([17, 18], 2, start_pos=prefill)  # a valid decode state at context prefill + 2
    return eng


def step_groups(eng):
    """The launch groups the step runs: Q/K/V, attention and the O projection
    as one group when the engine runs them as one launch (k_qkv_attn with its
    O phase; then the FFN as one group when it runs as k_ffn_xcd), Q/K/V and
    attention as one when only those are fused, else every group separately."""
    if eng.group_kernels("qkv_attn_o").count(";") == 0 and "k_qkv_attn" in eng.group_kernels("qkv_attn_o"):
        if "k_ffn_xcd" in eng.group_kernels("ffn") or "k_moe_xcd" in eng.group_kernels("ffn"):
            return ["qkv_attn_o", "ffn"]
        return ["qkv_attn_o"] + GROUP_ORDER[3:]
    if "k_qkv_attn" in eng.group_kernels("qkv_attn"):
        return ["qkv_attn"] + GROUP_ORDER[2:]
    return list(GROUP_ORDER)


def per_kernel(eng, L, iters=108):
    """{group: us, bytes, GB/s, frac} for every launch group, and the dominant one."""
    rows = {}
    for g in step_groups(eng):
        us = eng.time_kernel(g, iters)
        b = eng.group_bytes(g, L)
        gbs = b / (us * 1e-6) / 1e9
        rows[g] = {"kernel": eng.group_kernels(g), "us_per_launch": round(us, 3), "bytes_per_launch": b,
                   "achieved_GBs": round(gbs, 1), "frac": round(gbs / PEAK, 4)}
    dom = max(rows, key=lambda g: rows[g]["us_per_launch"])
    return rows, dom


def pmc_sequence(ctx, model=DENSE_8B, prefill=PREFILL):
    """Calibration read, calibration write, then every group's launches."""
    cal = ctx.alloc(CAL_BYTES)
    ctx.synth_vector(cal, 0, 1, CAL_BYTES // 2, 1.0, 7, 7)  # warm the pages (not used)
    eng = probe_engine(ctx, prefill + 64, model, prefill)
    ctx.sync()
    ctx.stream_read_probe(cal, CAL_BYTES, 1)             # k_stream_read: reads CAL_BYTES (twice: warm + timed)
    ctx.synth_vector(cal, 0, 0, CAL_BYTES // 4, 1.0, 8, 8)  # k_synth_vector: writes CAL_BYTES
    groups = step_groups(eng)
    for g in groups:
        eng.time_kernel(g, PMC_ITERS)
    ctx.sync()
    b = {g: eng.group_bytes(g, prefill + 2) for g in groups}
    eng.deinit()
    ctx.free(cal)
    return b


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--pmc", action="store_true", help="run the counter-calibration launch sequence")
    ap.add_argument("--config", type=int, choices=[3, 4], default=3, help="config 3 (dense 8B) or 4 (48-layer MoE)")
    a = ap.parse_args()
    model, prefill = (DENSE_8B, PREFILL) if a.config == 3 else (MOE_48L, PREFILL_C4)
    ctx = hip.Context(0)
    if a.pmc:
        b = pmc_sequence(ctx, model, prefill)
        print(json.dumps({"cal_bytes": CAL_BYTES, "groups": list(b), "iters": PMC_ITERS,
                          "layers": model["n_layers"], "alg_bytes": b, "config": a.config,
                          "context": prefill + 2}), flush=True)
    else:
        eng = probe_engine(ctx, prefill + 64, model, prefill)
        rows, dom = per_kernel(eng, prefill + 2)
        eng.deinit()
        print(json.dumps({"dominant": dom, "kernels": rows}), flush=True)
    ctx.close()
    return 0


if __name__ == "__main__":
    sys.exit(main())
