"""Turns two rocprofv3 counter runs of `python3 -m benchmarks.roofline_probe --pmc`
(FETCH_SIZE, then WRITE_SIZE; CSV output) into the per-launch HBM traffic of
every launch group of the decode step, calibrated against kernels of known
size in the same run:

    FETCH factor = bytes read by each k_stream_* launch / its FETCH_SIZE (KiB)
    WRITE factor = bytes written by the k_synth_vector calibration write
                   (its dispatches right after the reads) / their WRITE_SIZE (KiB)
    traffic      = FETCH_SIZE(kernel) * FETCH factor + WRITE_SIZE(kernel) * WRITE factor

    python -m benchmarks.pmc_summary FETCH_DIR WRITE_DIR PROBE_JSON OUT.md

PROBE_JSON is the probe's stdout (the groups, launches per group and each
group's algorithmic bytes). After the calibration write, the dispatches come
in group order, (layers + iters) per group. OUT.md records the commands, the
factors and the per-launch figures; its `traffic_bytes_per_launch[group]:`
lines are what bench.py reports as roofline.traffic.
"""
import csv
import glob
import json
import os
import statistics
import sys


def _rows(d):
    f = glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True)
    if not f:
        raise SystemExit(f"no counter_collection.csv under {d}")
    rows = list(csv.DictReader(open(f[0])))
    rows.sort(key=lambda r: int(r["Dispatch_Id"]))
    return rows


def _split(rows, groups, per_group):
    """Calibration dispatches and the per-group blocks after them."""
    # (the probe's three read patterns, each reading the calibration bytes)
    def is_read(r):
        return r["Kernel_Name"].removeprefix("void ").startswith("k_stream_")
    last_read = max(i for i, r in enumerate(rows) if is_read(r))
    cal_r = [float(r["Counter_Value"]) for r in rows if is_read(r)]
    after = rows[last_read + 1:]
    nw = 0  # the calibration write: the k_synth_vector dispatches right after the reads
    while nw < len(after) and after[nw]["Kernel_Name"].startswith("k_synth_vector"):
        nw += 1
    if nw == 0:
        raise SystemExit(f"expected the calibration write after the reads, got {after[0]['Kernel_Name']}")
    cal_w = sum(float(r["Counter_Value"]) for r in after[:nw])
    # the runtime's own copies / fills (reading results back) are not groups
    body = [r for r in after[nw:] if not r["Kernel_Name"].startswith("__amd_rocclr")]
    if len(body) != len(groups) * per_group:
        raise SystemExit(f"expected {len(groups)} x {per_group} dispatches after calibration, got {len(body)}")
    blocks = {g: body[i * per_group:(i + 1) * per_group] for i, g in enumerate(groups)}
    return cal_r, cal_w, blocks


def summarize(fetch_dir, write_dir, probe):
    groups, per = probe["groups"], probe["layers"] + probe["iters"]
    cal_bytes = probe["cal_bytes"]
    fr, _, fb = _split(_rows(fetch_dir), groups, per)
    _, cw, wb = _split(_rows(write_dir), groups, per)
    f_fetch = cal_bytes / (statistics.mean(fr) * 1024.0)
    f_write = cal_bytes / (cw * 1024.0)
    out = {"fetch_factor": f_fetch, "write_factor": f_write, "groups": {}}
    for g in groups:
        names = sorted({r["Kernel_Name"] for r in fb[g]})
        fk = statistics.mean(float(r["Counter_Value"]) for r in fb[g])
        wk = statistics.mean(float(r["Counter_Value"]) for r in wb[g])
        t = fk * 1024.0 * f_fetch + wk * 1024.0 * f_write
        out["groups"][g] = {"kernels": names, "fetch_kib": fk, "write_kib": wk, "traffic": t,
                            "alg_bytes": probe["alg_bytes"][g]}
    return out


def main():
    if len(sys.argv) != 5:
        print(__doc__)
        return 2
    probe = json.loads(open(sys.argv[3]).read().strip().splitlines()[-1])
    s = summarize(sys.argv[1], sys.argv[2], probe)
    cfg = probe.get("config", 3)
    sfx = "" if cfg == 3 else f" --config {cfg}"
    tag = "" if cfg == 3 else f"_c{cfg}"
    cmd = ("cd /tmp && export TMPDIR=/tmp && cd $GRAFT_REPO_ROOT && timeout -s KILL 180 rocprofv3 --pmc {c} "
           "-d gpurun_out/pmc_{d} -o run --output-format csv -- python3 -m benchmarks.roofline_probe --pmc" + sfx +
           " > gpurun_out/pmc_{d}.json")
    title = ("the 8B decode step's kernels (config 3)" if cfg == 3 else
             "the 48-layer MoE decode step's kernels (config 4)")
    with open(sys.argv[4], "w") as f:
        f.write(f"# HBM traffic per launch of {title}\n\n")
        f.write("Commands (one counter per run, from the repository root):\n\n")
        f.write("    " + cmd.format(c="FETCH_SIZE", d="fetch" + tag) + "\n")
        f.write("    " + cmd.format(c="WRITE_SIZE", d="write" + tag) + "\n")
        f.write(f"    python -m benchmarks.pmc_summary gpurun_out/pmc_fetch{tag} gpurun_out/pmc_write{tag} "
                f"gpurun_out/pmc_fetch{tag}.json <this file>\n\n")
        f.write("Calibration (kernels of known size in the same run):\n\n")
        f.write(f"- k_stream_read / k_stream_slice of {probe['cal_bytes']} B: FETCH_SIZE factor {s['fetch_factor']:.4f} "
                "(bytes = counter KiB x 1024 x factor)\n")
        f.write(f"- k_synth_vector write of {probe['cal_bytes']} B: WRITE_SIZE factor {s['write_factor']:.4f}\n\n")
        f.write(f"Per launch (mean over {probe['layers'] + probe['iters']} launches per group, rotating through "
                f"the {probe['layers']} layers; KV context {probe.get('context', 4098)}):\n\n")
        f.write("| group | kernel | FETCH_SIZE KiB | WRITE_SIZE KiB | traffic B | algorithmic B | traffic / alg |\n")
        f.write("|---|---|---|---|---|---|---|\n")
        for g, r in s["groups"].items():
            f.write(f"| {g} | `{', '.join(r['kernels'])}` | {r['fetch_kib']:.1f} | {r['write_kib']:.1f} | "
                    f"{r['traffic']:.0f} | {r['alg_bytes']} | {r['traffic'] / r['alg_bytes']:.4f} |\n")
        f.write("\n")
        for g, r in s["groups"].items():
            f.write(f"traffic_bytes_per_launch[{g}]: {r['traffic']:.0f}\n")
    print(open(sys.argv[4]).read())
    return 0


if __name__ == "__main__":
    sys.exit(main())
