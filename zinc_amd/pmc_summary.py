"""Turns two rocprofv3 counter runs of `python3 -m zinc_amd.roofline_probe --pmc`
(FETCH_SIZE, then WRITE_SIZE; CSV output) into the per-launch HBM traffic of
the dominant decode kernel, calibrated against kernels of known size:

    FETCH factor = bytes read by k_stream_read / its FETCH_SIZE (KiB)
    WRITE factor = bytes written by the k_synth_vector calibration write /
                   its WRITE_SIZE (KiB)
    traffic      = FETCH_SIZE(kernel) * FETCH factor + WRITE_SIZE(kernel) * WRITE factor

    python -m zinc_amd.pmc_summary FETCH_DIR WRITE_DIR OUT.md

OUT.md records the commands, the factors and the per-launch figures; its
`traffic_bytes_per_launch:` line is what bench.py reports as roofline.traffic.
"""
import csv
import glob
import os
import statistics
import sys

from .roofline_probe import CAL_BYTES, down_bytes

KERNEL = "k_dmmv_q6k_tile<128"


def _rows(d):
    f = glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True)
    if not f:
        raise SystemExit(f"no counter_collection.csv under {d}")
    return list(csv.DictReader(open(f[0])))


def summarize(fetch_dir, write_dir):
    fr, wr = _rows(fetch_dir), _rows(write_dir)
    # calibration read: the k_stream_read dispatches (CAL_BYTES each)
    cal_r = [float(r["Counter_Value"]) for r in fr if r["Kernel_Name"].startswith("k_stream_read")]
    # calibration write: the k_synth_vector dispatches after the reads (CAL_BYTES in total)
    ids = [int(r["Dispatch_Id"]) for r in wr if r["Kernel_Name"].startswith("k_stream_read")]
    last_read = max(ids)
    first_down = min(int(r["Dispatch_Id"]) for r in wr if KERNEL in r["Kernel_Name"])
    cal_w = sum(float(r["Counter_Value"]) for r in wr
                if r["Kernel_Name"].startswith("k_synth_vector") and last_read < int(r["Dispatch_Id"]) < first_down)
    f_fetch = CAL_BYTES / (statistics.mean(cal_r) * 1024.0)
    f_write = CAL_BYTES / (cal_w * 1024.0)
    kf = [float(r["Counter_Value"]) for r in fr if KERNEL in r["Kernel_Name"]]
    kw = [float(r["Counter_Value"]) for r in wr if KERNEL in r["Kernel_Name"]]
    fetch_b = statistics.mean(kf) * 1024.0 * f_fetch
    write_b = statistics.mean(kw) * 1024.0 * f_write
    return {"fetch_factor": f_fetch, "write_factor": f_write, "fetch_kib": statistics.mean(kf),
            "write_kib": statistics.mean(kw), "launches": len(kf), "fetch_bytes": fetch_b,
            "write_bytes": write_b, "traffic": fetch_b + write_b, "alg_bytes": down_bytes()[1]}


def main():
    if len(sys.argv) != 4:
        print(__doc__)
        return 2
    s = summarize(sys.argv[1], sys.argv[2])
    cmd = ("cd /tmp && export TMPDIR=/tmp && cd $GRAFT_REPO_ROOT && timeout -s KILL 90 rocprofv3 --pmc {c} "
           "-d gpurun_out/pmc_{d} -o run --output-format csv -- python3 -m zinc_amd.roofline_probe --pmc")
    with open(sys.argv[3], "w") as f:
        f.write(f"# HBM traffic of {KERNEL} (ffn_down, Q6_K 4096x12288, y += W x)\n\n")
        f.write("Commands (one counter per run, from the repository root):\n\n")
        f.write("    " + cmd.format(c="FETCH_SIZE", d="fetch") + "\n")
        f.write("    " + cmd.format(c="WRITE_SIZE", d="write") + "\n")
        f.write("    python -m zinc_amd.pmc_summary gpurun_out/pmc_fetch gpurun_out/pmc_write <this file>\n\n")
        f.write("Calibration (kernels of known size in the same run):\n\n")
        f.write(f"- k_stream_read of {CAL_BYTES} B: FETCH_SIZE factor {s['fetch_factor']:.4f} (bytes = counter KiB x 1024 x factor)\n")
        f.write(f"- k_synth_vector write of {CAL_BYTES} B: WRITE_SIZE factor {s['write_factor']:.4f}\n\n")
        f.write(f"Per launch (mean of {s['launches']} launches over 14 rotating weight copies, 578 MB):\n\n")
        f.write(f"- FETCH_SIZE {s['fetch_kib']:.1f} KiB -> {s['fetch_bytes']:.0f} B\n")
        f.write(f"- WRITE_SIZE {s['write_kib']:.1f} KiB -> {s['write_bytes']:.0f} B\n")
        f.write(f"- algorithmic bytes {s['alg_bytes']} (weights + x + y read/write)\n")
        f.write(f"- traffic / algorithmic = {s['traffic'] / s['alg_bytes']:.4f}\n\n")
        f.write(f"traffic_bytes_per_launch: {s['traffic']:.0f}\n")
    print(open(sys.argv[3]).read())
    return 0


if __name__ == "__main__":
    sys.exit(main())
