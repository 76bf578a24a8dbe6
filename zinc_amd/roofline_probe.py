"""Roofline measurement of the decode step's dominant kernel, and the launch
sequence its hardware-counter profile is taken from.

The dominant kernel of the 8B-shape decode step (largest share of step time
in the kernel-trace profile) is the ffn_down projection: Q6_K 4096 x 12288
with the f32 SwiGLU output staged in every workgroup and the residual added
in place (acc_mode 1), i.e. `dispatchDmmvAcc` at forward.zig:7420 with
dmmv_q6k.comp. Its algorithmic bytes per launch are the weight blocks, the
activation and the read-modify-write of y.

    python -m zinc_amd.roofline_probe            # timing only
    rocprofv3 --pmc FETCH_SIZE -- python3 -m zinc_amd.roofline_probe --pmc

With --pmc the script launches, in order: a streaming read of CAL_BYTES
(cold, known size), a write of CAL_BYTES (known size), then PMC_LAUNCHES
launches of the down projection; the counter of each launch is read from
the profiler output and the first two give the bytes-per-counter factors.
"""
import argparse
import json
import sys

from . import hip

M_DOWN, K_DOWN = 4096, 12288
N_COPIES = 14            # 14 x 41.3 MB = 578 MB of distinct weights > 256 MB MALL
CAL_BYTES = 1 << 30      # calibration read / write size
PMC_LAUNCHES = 20


def down_bytes():
    wb = hip.tensor_bytes(hip.Q6_K, M_DOWN, K_DOWN)
    return wb, wb + K_DOWN * 4 + 2 * M_DOWN * 4


class DownProjection:
    """N_COPIES seeded weight copies, the activation and the output."""

    def __init__(self, ctx):
        self.ctx = ctx
        self.wb, self.alg_bytes = down_bytes()
        self.W = ctx.alloc(self.wb * N_COPIES)
        for i in range(N_COPIES):
            ctx.synth_tensor(self.W, i * self.wb, hip.Q6_K | 0x100, M_DOWN, K_DOWN, 4242, 300 + i)
        self.x = ctx.alloc(K_DOWN * 4)
        ctx.synth_vector(self.x, 0, 0, K_DOWN, 1.0, 4242, 299)
        self.y = ctx.alloc(M_DOWN * 4)
        ctx.synth_vector(self.y, 0, 0, M_DOWN, 1.0, 4242, 298)

    def launch(self, i):
        c = i % N_COPIES
        self.ctx.dmmv(hip.Q6_K, self.W, c * self.wb, self.x, 0, self.y, 0, M_DOWN, K_DOWN, 1)

    def close(self):
        for b in (self.W, self.x, self.y):
            self.ctx.free(b)


def time_dominant_kernel(ctx, iters=200):
    """Average launch duration (HIP events on the library stream) and the
    achieved algorithmic GB/s of the down projection."""
    d = DownProjection(ctx)
    for i in range(2 * N_COPIES):
        d.launch(i)
    ctx.sync()
    ctx.record(0)
    for i in range(iters):
        d.launch(i)
    ctx.record(1)
    ms = ctx.elapsed_ms(0, 1)
    d.close()
    us = ms * 1e3 / iters
    return {"kernel": "k_dmmv_q6k_tile<128> (ffn_down, Q6_K 4096x12288, f32 x staged per workgroup, y += W x)",
            "us_per_launch": round(us, 3), "bytes_per_launch": d.alg_bytes,
            "achieved_GBs": round(d.alg_bytes / (us * 1e-6) / 1e9, 1)}


def pmc_sequence(ctx):
    """Calibration read, calibration write, then PMC_LAUNCHES down launches."""
    cal = ctx.alloc(CAL_BYTES)
    ctx.synth_vector(cal, 0, 1, CAL_BYTES // 2, 1.0, 7, 7)  # warm the pages (not used)
    d = DownProjection(ctx)
    ctx.sync()
    ctx.stream_read_probe(cal, CAL_BYTES, 1)             # k_stream_read: reads CAL_BYTES (twice: warm + timed)
    ctx.synth_vector(cal, 0, 0, CAL_BYTES // 4, 1.0, 8, 8)  # k_synth_vector: writes CAL_BYTES
    for i in range(PMC_LAUNCHES):
        d.launch(i)
    ctx.sync()
    d.close()
    ctx.free(cal)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--pmc", action="store_true", help="run the counter-calibration launch sequence")
    a = ap.parse_args()
    ctx = hip.Context(0)
    if a.pmc:
        pmc_sequence(ctx)
        print(json.dumps({"cal_bytes": CAL_BYTES, "down_launches": PMC_LAUNCHES,
                          "alg_bytes": down_bytes()[1]}), flush=True)
    else:
        print(json.dumps(time_dominant_kernel(ctx)), flush=True)
    ctx.close()
    return 0


if __name__ == "__main__":
    sys.exit(main())
