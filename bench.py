"""Headline benchmark: batch-1 greedy decode of the 8B-shaped Q4_K_M model
on one MI355X, plus the roofline of the dominant kernel
and the CPU oracle timed on the host beside it.

python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu-baseline]

Prints ONE JSON line on stdout.
"""
import argparse
import json
import os
import re
import subprocess
import sys
import tempfile
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_HBM_GBS = 8000.0  # MI355X published HBM3E bandwidth
PREFILL = 4096          # KV context pre-filled before the prompt (config 3)
N_PROMPT = 16


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def stream_ceiling(ctx, nbytes=1 << 30):
    """Measured streaming-read rate (zh_stream_read_probe: the counterpart of
    the reference's bandwidth microbenchmark) over nbytes, in GB/s."""
    buf = ctx.alloc(nbytes)
    ctx.synth_vector(buf, 0, 1, nbytes // 2, 1.0, 7, 7)  # touch the pages
    gbs = ctx.stream_read_probe(buf, nbytes, 10)
    ctx.free(buf)
    return gbs


def kernel_roofline(eng, L):
    """Per-kernel bandwidth of every per-layer launch group of the decode step
    (benchmarks.roofline_probe: the engine replays its own launches with HIP
    events on its stream, rotating through the layers) and the roofline of the
    dominant one (largest launch duration = largest share of step time).
    `traffic` is the counter-measured HBM bytes per launch of that group from
    profiles/decode_kernels_pmc.md."""
    from benchmarks import roofline_probe
    rows, dom = roofline_probe.per_kernel(eng, L)
    r = rows[dom]
    traffic = None
    pm = os.path.join(ROOT, "profiles", "decode_kernels_pmc.md")
    if os.path.exists(pm):
        m = re.search(r"^traffic_bytes_per_launch\[%s\]: (\d+)" % dom, open(pm).read(), re.M)
        traffic = int(m.group(1)) if m else None
    roof = {"kernel": eng.group_kernels(dom), "bound": "hbm", "achieved": r["achieved_GBs"], "peak": PEAK_HBM_GBS,
            "unit": "GB/s", "frac": r["frac"], "traffic": traffic, "bytes_per_launch": r["bytes_per_launch"],
            "us_per_launch": r["us_per_launch"], "group": dom}
    per = {g: {"us": v["us_per_launch"], "GBs": v["achieved_GBs"], "frac": v["frac"]} for g, v in rows.items()}
    return roof, per


def cpu_baseline(cfg, n_tokens=16):
    """The CPU oracle (C restatement of the reference's dequantRow + serial f32
    dot path, threaded over rows as forward_metal.zig:3932-3933) decoding
    `n_tokens` tokens of the same model at position PREFILL."""
    # the baseline runs a build for this host's own CPU (BASELINE's -march=native),
    # made here from the committed source; the shipped x86-64-v3 copy if that fails
    native = os.path.join(tempfile.gettempdir(), f"zo_native_{os.getpid()}", "libzinc_oracle.so")
    os.makedirs(os.path.dirname(native), exist_ok=True)
    mk = subprocess.run(["make", "-s", "-C", os.path.join(ROOT, "oracle"), "MARCH=native", f"OUT={native}"],
                        capture_output=True, text=True)
    march = "native" if mk.returncode == 0 and os.path.exists(native) else "x86-64-v3"
    if march == "native":
        os.environ["ZO_LIB_PATH"] = native
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as orc
    nproc = os.cpu_count() or 1
    threads = min(nproc, 16)
    t0 = time.time()
    om = orc.Model(cfg, nthreads=threads)
    om.prefill_kv_random(PREFILL, 7)
    build_s = time.time() - t0
    t0 = time.time()
    tok = 17
    for i in range(n_tokens):
        tok = om.decode_step(tok, PREFILL + i)
    dt = time.time() - t0
    om.close()
    return {"value": round(n_tokens / dt, 4), "unit": "tok/s", "cores": threads, "threads": threads,
            "nproc": nproc, "kind": "port",
            "sample": f"{n_tokens} greedy decode steps of the same 8B-shaped model at context {PREFILL} "
                      f"(oracle built with -march={march}; model build {build_s:.0f}s untimed)"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=256)
    ap.add_argument("--warmup", type=int, default=16)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-tokens", type=int, default=16)
    ap.add_argument("--pages", choices=["ident", "shuffle"], default="ident",
                    help="KV page table: identity, or a seeded permutation (the paged attention kernel)")
    ap.add_argument("--persistent", type=int, default=0,
                    help="1: the step's layers in one persistent launch (zh_engine_set_persistent)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (this build has no multi-GPU path); got --gpus {args.gpus}",
              file=sys.stderr)
        sys.exit(2)

    import zinc_amd
    cfg = dict(zinc_amd.DENSE_8B)
    cfg["max_ctx"] = PREFILL + N_PROMPT + args.warmup + args.steps + 16
    cfg["max_ctx"] = (cfg["max_ctx"] + 15) // 16 * 16
    ctx = zinc_amd.Context(0)
    name, cus, hbm = ctx.info()
    log(f"device: {name}, {cus} CUs, {hbm / 2**30:.0f} GiB")
    t0 = time.time()
    eng = zinc_amd.InferenceEngine(ctx, cfg)
    if args.pages == "shuffle":
        eng.set_pages(np.random.default_rng(17).permutation(cfg["max_ctx"] // 16).astype(np.uint32))
    eng.set_persistent(bool(args.persistent))
    eng.prefill_kv_random(PREFILL, 7)
    ctx.sync()
    log(f"engine init + synthetic weights + KV prefill: {time.time() - t0:.1f}s")

    rng = np.random.default_rng(1234)
    prompt = [int(t) for t in rng.integers(0, cfg["vocab"], N_PROMPT)]
    # warmup: prompt + W greedy tokens (also captures the step graphs)
    warm = eng.generate(prompt, max(args.warmup, 1), start_pos=PREFILL)
    pos = PREFILL + N_PROMPT + len(warm) - 1
    ctx.sync()
    # timed: exactly K decode steps (one token each), fed back on device
    t0 = time.perf_counter()
    ctx.record(10)
    toks = eng.generate([warm[-1]], args.steps, start_pos=pos)
    ctx.record(11)
    ctx.sync()
    wall = time.perf_counter() - t0
    gpu_ms = ctx.elapsed_ms(10, 11)
    ms_per_step = wall * 1e3 / args.steps
    L_mid = pos + args.steps // 2
    bytes_tok = eng.bytes_per_token(L_mid)
    tok_s = args.steps / wall
    log(f"decode: {tok_s:.1f} tok/s ({ms_per_step:.3f} ms/token wall, {gpu_ms / args.steps:.3f} ms/token GPU), "
        f"{bytes_tok / 1e9:.3f} GB/token -> {bytes_tok * tok_s / 1e9:.0f} GB/s "
        f"({bytes_tok * tok_s / 1e9 / PEAK_HBM_GBS:.1%} of 8 TB/s); distinct tokens {len(set(toks))}")

    # per-kernel bandwidth (after the timed region; it changes the activations)
    roof, per_kernel = kernel_roofline(eng, pos + args.steps)
    # consistency of the isolated group replays with the graph-replayed step:
    # layers x (sum of the groups' launch durations) + the head, against the
    # step time measured around the timed graph replays
    L = cfg["n_layers"]
    step_from_groups = L * sum(v["us"] for v in per_kernel.values()) + eng.head_us()
    per_kernel_graph = {"step_us_graph": round(gpu_ms / args.steps * 1e3, 1),
                        "step_us_from_isolated_groups": round(step_from_groups, 1)}
    ceiling = stream_ceiling(ctx)
    roof["stream_ceiling"] = round(ceiling, 1)
    roof["frac_of_stream_ceiling"] = round(roof["achieved"] / ceiling, 4)
    log(f"dominant kernel ({roof['group']}): {roof['achieved']} GB/s ({roof['frac']:.1%}, "
        f"{roof['frac_of_stream_ceiling']:.1%} of the {ceiling:.0f} GB/s stream ceiling), "
        f"{roof['us_per_launch']} us/launch; per kernel: {per_kernel}; step vs groups: {per_kernel_graph}")
    eng.deinit()
    ctx.close()

    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_baseline(cfg, args.cpu_tokens)
        log(f"cpu baseline: {cpu}")

    out = {
        "metric": "decode tok/s, 8B-shape Q4_K_M bs=1; DMMV HBM GB/s vs 8 TB/s peak",
        "value": round(tok_s, 2), "unit": "tok/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "q4_k/q6_k weights, int8-limb dot4 + f32 accumulate, fp16 KV",
        "data": "synthetic (seeded random-init weights, N(0,1) fp16 KV prefill)",
        "config": {"workload": "config 3: dense 8B-shape decoder (36L, 4096 hidden, 32q/8kv heads, ffn 12288, "
                               "vocab 151936), Q4_K_M, batch 1, greedy decode at KV context 4096+",
                   "context_start": pos, "bytes_per_token": bytes_tok,
                   "token_roofline_frac": round(bytes_tok * tok_s / 1e9 / PEAK_HBM_GBS, 4),
                   "token_frac_of_stream_ceiling": round(bytes_tok * tok_s / 1e9 / ceiling, 4),
                   "gpu_ms_per_step": round(gpu_ms / args.steps, 4),
                   "kv_pages": args.pages, "persistent_layers": bool(args.persistent),
                   "residual_sums": "64-bit fixed point (bit-reproducible decode)"},
        "roofline": roof,
        "per_kernel": per_kernel,
        "step_consistency": per_kernel_graph,
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
