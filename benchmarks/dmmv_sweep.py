"""Configs 1-2 measurement: one DMMV launch per shape at batch 1, timed with
HIP events on the library stream over a rotating set of weight copies larger
than the 256 MB MALL (so every launch streams its weights from HBM), as the
reference's bench_hot_decode rotates a 16-slot working set.

    python -m benchmarks.dmmv_sweep [--iters 60] [--md OUT.md]

Per shape: zh_dmmv (f32 activation, the C-ABI entry that replaces
DmmvDispatch.recordDispatch, dmmv.zig:806-874) and zh_dmmv_xq (the
activation pre-quantised once, as the engine feeds the projections that share
an input). Algorithmic bytes = weight blocks + 4 K (x) + 4 M (y), the
per-kernel figure of the bandwidth roofline; fraction of the 8 TB/s peak.
A streaming read of 1 GiB gives the measured ceiling beside it.

    python -m benchmarks.dmmv_sweep --batched [--md OUT.md]

Under rocprofv3 --kernel-trace, each timed block of launches is bracketed by
two four-element k_swiglu launches (separators), so

    python -m benchmarks.dmmv_sweep --from-trace RUN_kernel_trace.csv SWEEP.json [--md OUT.md]

recovers every (shape, activation) entry's kernel time per call from the
trace: per kernel of the call, the mean of the middle 80% of its dispatch
durations, summed over the kernels the call launches.

instead times the batched DMMV (zh_dmmv_batched / the gate/up form, the
skinny GEMM of recordBatchDispatchPush, dmmv.zig:880-925) on the config-3
decode shapes at 1, 2, 4 and 8 activation vectors: microseconds per launch
and the weight bytes streamed per vector-microsecond (the one-vector rate
times the speed-up over one launch per vector).
"""
import argparse
import json
import statistics
import sys

from zinc_amd import hip

PEAK = 8000.0  # GB/s
ROTATE_BYTES = 600 << 20

SHAPES = [
    ("config 1: Q4_K 4096x4096", hip.Q4_K, 4096, 4096),
    ("Q4_K 4096->12288 (gate/up)", hip.Q4_K, 12288, 4096),
    ("Q4_K 12288->4096 (down)", hip.Q4_K, 4096, 12288),
    ("Q6_K 4096->151936 (lm-head)", hip.Q6_K, 151936, 4096),
    ("Q5_K 4096x4096", hip.Q5_K, 4096, 4096),
    ("Q5_K 4096->12288 (gate/up)", hip.Q5_K, 12288, 4096),
    ("Q5_K 12288->4096 (down)", hip.Q5_K, 4096, 12288),
    ("Q8_0 4096x4096", hip.Q8_0, 4096, 4096),
    ("MXFP4 2880x2880", hip.MXFP4, 2880, 2880),
]


def measure(ctx, name, qt, M, K, iters):
    wb = hip.tensor_bytes(qt, M, K)
    ncp = max(2, -(-ROTATE_BYTES // wb))
    W = ctx.alloc(wb * ncp)
    for i in range(ncp):
        ctx.synth_tensor(W, i * wb, qt, M, K, 1234 + 2, 100 + i)
    x = ctx.alloc(K * 4)
    ctx.synth_vector(x, 0, 0, K, 1.0, 1234 + 2, 99)
    xq = ctx.alloc(ctx.xq_bytes(K))
    ctx.quantize_activation(x, 0, K, xq)
    y = ctx.alloc(M * 4)
    sep = ctx.alloc(256)
    alg = wb + 4 * K + 4 * M
    res = {"shape": name, "qtype": qt, "M": M, "K": K, "weight_bytes": wb, "alg_bytes": alg, "copies": ncp}
    for label, fn in (("f32_x", lambda c: ctx.dmmv(qt, W, c * wb, x, 0, y, 0, M, K, 0)),
                      ("xq_x", lambda c: ctx.dmmv_xq(qt, W, c * wb, xq, 0, y, 0, M, K, 0))):
        try:
            fn(0)
        except hip.ZincError as e:  # a format without an XQ-input kernel
            res[label] = {"error": e.name}
            continue
        for i in range(2 * ncp):
            fn(i % ncp)
        ctx.sync()
        ctx.swiglu(sep, sep, sep, 4)  # separator (kernel trace: the sweep launches no other k_swiglu)
        ctx.record(0)
        for i in range(iters):
            fn(i % ncp)
        ctx.record(1)
        ctx.swiglu(sep, sep, sep, 4)
        ctx.sync()
        us = ctx.elapsed_ms(0, 1) * 1e3 / iters
        gbs = alg / (us * 1e-6) / 1e9
        res[label] = {"us": round(us, 3), "GBs": round(gbs, 1), "frac": round(gbs / PEAK, 4)}
    for b in (W, x, xq, y, sep):
        ctx.free(b)
    return res


def from_trace(csv_path, sweep_json):
    """Per (shape, activation) entry: the kernels between each pair of
    separators and their time per call (middle-80% mean per kernel, summed).
    Given a counter-collection CSV (rocprofv3 --pmc FETCH_SIZE) instead: the
    fetched bytes per call, calibrated against the sweep's 1 GiB stream
    probe (k_stream_read / k_stream_slice) in the same run."""
    import csv
    rows = list(csv.DictReader(open(csv_path)))
    pmc = "Counter_Value" in rows[0]
    rows.sort(key=lambda r: int(r["Dispatch_Id"] if pmc else r["Start_Timestamp"]))
    factor = 1.0
    if pmc:
        cal = [float(r["Counter_Value"]) for r in rows if r["Kernel_Name"].removeprefix("void ").startswith("k_stream_")]
        factor = (1 << 30) / (statistics.mean(cal) * 1024.0)
    sweep = json.loads(open(sweep_json).read().strip().splitlines()[-1])
    entries = [(r["shape"], lab) for r in sweep["shapes"] for lab in ("f32_x", "xq_x") if "us" in r[lab]]
    seps = [i for i, r in enumerate(rows) if "k_swiglu" in r["Kernel_Name"]]
    if len(seps) != 2 * len(entries):
        raise SystemExit(f"expected {2 * len(entries)} separators, found {len(seps)}")
    out = []
    for k, (shape, lab) in enumerate(entries):
        block = rows[seps[2 * k] + 1:seps[2 * k + 1]]
        by = {}
        for r in block:
            v = (float(r["Counter_Value"]) * 1024.0 * factor if pmc
                 else (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3)
            by.setdefault(r["Kernel_Name"], []).append(v)
        calls = max(len(v) for v in by.values())
        us, names = 0.0, []
        for name, d in by.items():
            d = sorted(d)
            cut = len(d) // 10
            mid = d[cut:len(d) - cut] or d
            us += sum(mid) / len(mid) * len(d) / calls
            names.append(name.split("(")[0])
        alg = next(r["alg_bytes"] for r in sweep["shapes"] if r["shape"] == shape)
        if pmc:  # (us holds bytes here)
            out.append({"shape": shape, "entry": lab, "kernels": names, "fetch_bytes": round(us),
                        "alg_bytes": alg, "fetch_over_alg": round(us / alg, 4)})
        else:
            out.append({"shape": shape, "entry": lab, "kernels": names, "us": round(us, 3),
                        "frac": round(alg / (us * 1e-6) / 1e9 / PEAK, 4), "alg_bytes": alg})
    return out


BATCH_SHAPES = [
    ("Q/K/V Q4_K 6144x4096", hip.Q4_K, 6144, 4096, False),
    ("O Q4_K 4096x4096", hip.Q4_K, 4096, 4096, False),
    ("gate/up Q4_K 2 x 12288x4096 + SwiGLU", hip.Q4_K, 12288, 4096, True),
    ("down Q6_K 4096x12288", hip.Q6_K, 4096, 12288, False),
    ("LM head Q6_K 151936x4096", hip.Q6_K, 151936, 4096, False),
]


def measure_batched(ctx, name, qt, M, K, gate_up, ncols=(1, 2, 4, 8), iters=40):
    wb = hip.tensor_bytes(qt, M, K)
    nm = 2 if gate_up else 1
    ncp = max(2, -(-ROTATE_BYTES // (wb * nm)))
    W = ctx.alloc(wb * nm * ncp)
    for i in range(nm * ncp):
        ctx.synth_tensor(W, i * wb, qt | (0x100 if qt == hip.Q4_K else 0), M, K, 1234 + 3, 100 + i)
    nmax = max(ncols)
    X = ctx.alloc(4 * K * nmax)
    ctx.synth_vector(X, 0, 0, K * nmax, 1.0, 1234 + 3, 99)
    Y = ctx.alloc(4 * M * nmax)
    res = {"shape": name, "qtype": qt, "M": M, "K": K, "weight_bytes": wb * nm, "cols": {}}
    for n in ncols:
        def fn(c):
            if gate_up:
                ctx.dmmv_fused_gate_up_swiglu_batched(qt, W, 2 * c * wb, W, (2 * c + 1) * wb, X, 0, Y, 0, M, K, n)
            else:
                ctx.dmmv_batched(qt, W, c * wb, X, 0, Y, 0, M, K, n)
        for i in range(2 * ncp):
            fn(i % ncp)
        ctx.sync()
        ctx.swiglu(sep, sep, sep, 4)  # separator (kernel trace: the sweep launches no other k_swiglu)
        ctx.record(0)
        for i in range(iters):
            fn(i % ncp)
        ctx.record(1)
        ctx.swiglu(sep, sep, sep, 4)
        ctx.sync()
        us = ctx.elapsed_ms(0, 1) * 1e3 / iters
        res["cols"][n] = {"us": round(us, 2), "us_per_col": round(us / n, 2)}
    for b in (W, X, Y):
        ctx.free(b)
    return res


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--batched", action="store_true", help="time the batched DMMV at 1, 2, 4, 8 vectors")
    ap.add_argument("--iters", type=int, default=60)
    ap.add_argument("--md", default=None, help="also write a markdown table here")
    ap.add_argument("--from-trace", nargs=2, metavar=("TRACE_CSV", "SWEEP_JSON"),
                    help="kernel times per entry from a kernel trace of a sweep run")
    a = ap.parse_args()
    if a.from_trace:
        rows = from_trace(*a.from_trace)
        print(json.dumps(rows))
        if a.md:
            with open(a.md, "w") as f:
                if "us" in rows[0]:
                    f.write("| shape | activation | kernels | alg bytes | us per call | of 8 TB/s |\n"
                            "|---|---|---|---|---|---|\n")
                    for r in rows:
                        f.write(f"| {r['shape']} | {r['entry']} | `{' + '.join(r['kernels'])}` | {r['alg_bytes']:,} | "
                                f"{r['us']} | {r['frac']:.1%} |\n")
                else:
                    f.write("| shape | activation | kernels | alg bytes | FETCH bytes per call | fetch / alg |\n"
                            "|---|---|---|---|---|---|\n")
                    for r in rows:
                        f.write(f"| {r['shape']} | {r['entry']} | `{' + '.join(r['kernels'])}` | {r['alg_bytes']:,} | "
                                f"{r['fetch_bytes']:,} | {r['fetch_over_alg']:.3f} |\n")
        return 0
    ctx = hip.Context(0)
    if a.batched:
        rows = [measure_batched(ctx, *s) for s in BATCH_SHAPES]
        ctx.close()
        print(json.dumps({"workload": "batched DMMV on config-3 decode shapes, rotating weight copies > 256 MB MALL",
                          "shapes": rows}), flush=True)
        if a.md:
            with open(a.md, "w") as f:
                f.write("| shape | 1 col: us | 2 cols: us (per col) | 4 cols: us (per col) | 8 cols: us (per col) | "
                        "speed-up at 4 cols |\n|---|---|---|---|---|---|\n")
                for r in rows:
                    c = r["cols"]
                    f.write(f"| {r['shape']} | {c[1]['us']} | {c[2]['us']} ({c[2]['us_per_col']}) | "
                            f"{c[4]['us']} ({c[4]['us_per_col']}) | {c[8]['us']} ({c[8]['us_per_col']}) | "
                            f"{c[1]['us'] / c[4]['us_per_col']:.2f}x |\n")
        return 0
    cal = ctx.alloc(1 << 30)
    ctx.synth_vector(cal, 0, 1, (1 << 30) // 2, 1.0, 7, 7)
    stream_gbs = ctx.stream_read_probe(cal, 1 << 30, 3)
    ctx.free(cal)
    rows = [measure(ctx, *s, a.iters) for s in SHAPES]
    ctx.close()
    out = {"workload": "configs 1-2: single DMMV launches at batch 1, rotating weight copies > 256 MB MALL",
           "peak_GBs": PEAK, "stream_read_GBs": round(stream_gbs, 1), "shapes": rows}
    print(json.dumps(out), flush=True)
    if a.md:
        with open(a.md, "w") as f:
            f.write("| shape | alg bytes | f32 x: us | GB/s | of 8 TB/s | XQ x: us | GB/s | of 8 TB/s |\n")
            f.write("|---|---|---|---|---|---|---|---|\n")
            def cells(m):
                return f"{m['us']} | {m['GBs']} | {m['frac']:.1%}" if "us" in m else f"{m['error']} | - | -"
            for r in rows:
                f.write(f"| {r['shape']} | {r['alg_bytes']:,} | {cells(r['f32_x'])} | {cells(r['xq_x'])} |\n")
            f.write(f"\nStreaming read of 1 GiB (k_stream_read): {stream_gbs:.0f} GB/s.\n")
    return 0


if __name__ == "__main__":
    sys.exit(main())
