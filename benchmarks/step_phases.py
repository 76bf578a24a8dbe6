"""Per-workgroup timelines of the decode step's phases, from the debug
build's s_memrealtime trace points (100 MHz clock):

  - the persistent decode-layers kernel (zh_engine_set_persistent): start and
    end of each of layer 10's five phases in every workgroup, and the start
    of layer 11 (grid barrier + next-phase prefetch in the gaps);
  - the attention body inside it: its own trace points, relative to each
    workgroup's start (small copies landed, q fragments, ring steps,
    partials, merge).

Build the debug library first (it also compiles the points in):

    python -m zinc_amd.build --debug build/debug
    ZH_LIB_PATH=build/debug/libzinc_hip.so python -m benchmarks.step_phases
    ZH_LIB_PATH=build/debug/libzinc_hip.so python -m benchmarks.step_phases --standalone

--qkv-attn [--ctx N]: the Q/K/V + attention launch (k_qkv_attn) of the
per-phase step, replayed by zh_engine_time_kernel (KV context N, default
4096).

--ffn: the per-XCD FFN launch (k_ffn_xcd).

--moe: the per-XCD MoE FFN launch of config 4's model (k_moe_xcd).

--moe-attn: the attention launch of config 4's model (4 kv heads, 8 q heads
each, identity pages, KV context 8192).

--standalone: the same attention body as its own kernel (the per-phase
step with a shuffled page table, i.e. k_attn_ring), its launches replayed by
zh_engine_time_kernel; points relative to each workgroup's start.

Config 3's model (8B shapes, KV context 4096 + 2 decoded tokens).
"""
import ctypes as C
import os
import sys

import numpy as np

from zinc_amd import hip
from zinc_amd.engine import DENSE_8B, MOE_48L, InferenceEngine

ATTN_POINTS = {1: "small copies landed", 9: "q fragments", 10: "new K/V row ready", 5: "ring step 0 start",
               6: "ring step 0 end", 7: "ring step 1 start", 8: "ring step 1 end", 2: "after the ring",
               3: "partials stored", 4: "merger: start", 11: "merger: merge start", 12: "merger: stats",
               13: "merger: output"}


def print_attn(ta):
    ok = ta[:, 0] > 0
    for s in sorted(ATTN_POINTS, key=lambda k: [1, 9, 10, 5, 6, 7, 8, 2, 3, 4, 11, 12, 13].index(k)):
        col, st = ta[ok, s], ta[ok, 0]
        m = col >= st  # points the workgroup reached in this launch
        if not m.any():
            continue
        r = (col[m] - st[m]) * 0.01
        print(f"  {ATTN_POINTS[s]:22s}: n={m.sum():3d}  min {r.min():6.2f}  p50 {np.median(r):6.2f}  max {r.max():6.2f}")


def standalone(moe=False):
    L = hip.lib()
    L.zh_debug_trace_ops.argtypes = [C.POINTER(C.c_uint64), C.c_uint32]
    ctx = hip.Context(0)
    cfg = dict(MOE_48L if moe else DENSE_8B)
    ctxlen = 8192 if moe else 4096
    cfg["max_ctx"] = ctxlen + 64
    eng = InferenceEngine(ctx, cfg)
    if not moe:
        eng.set_pages(np.random.default_rng(17).permutation(cfg["max_ctx"] // 16).astype(np.uint32))
    eng.prefill_kv_random(ctxlen, 7)
    eng.generate([17, 18], 2, start_pos=ctxlen)
    ctx.sync()
    n = 8192 * 16
    a = np.zeros(n, np.uint64)
    L.zh_debug_trace_ops(a.ctypes.data_as(C.POINTER(C.c_uint64)), n)  # clears the points
    us = eng.time_kernel("attn", 36)
    ctx.sync()
    L.zh_debug_trace_ops(a.ctypes.data_as(C.POINTER(C.c_uint64)), n)
    print(f"standalone attention ({eng.group_kernels('attn')}): {us:.2f} us per launch (events, debug build); "
          "points of the last launch, us from each workgroup's start:")
    print_attn(a.reshape(8192, 16)[:ctx.info()[1]].astype(np.int64))
    eng.deinit()
    ctx.close()


QA_POINTS = ["start", "x landed", "XQ limbs in registers", "weight rows landed", "rows computed",
             "rows published", "rows of the head seen", "q, k, v, K/V landed", "q fragments", "scores and P V done",
             "partials published", "merger: chunks seen", "merger: output", "O rows added",
             "merge: start", "merge: statistics done"]


def qkv_attn(ctxlen=4096):
    """Per-workgroup timeline of k_qkv_attn (Q/K/V + attention in one launch)
    at a KV context of ctxlen (+ 2 decoded tokens)."""
    L = hip.lib()
    L.zh_debug_trace_qa.argtypes = [C.POINTER(C.c_uint64), C.c_uint32]
    ctx = hip.Context(0)
    cfg = dict(DENSE_8B)
    cfg["max_ctx"] = ctxlen + 64
    eng = InferenceEngine(ctx, cfg)
    eng.prefill_kv_random(ctxlen, 7)
    eng.generate([17, 18], 2, start_pos=ctxlen)
    ctx.sync()
    n = 8192 * 16
    a = np.zeros(n, np.uint64)
    L.zh_debug_trace_qa(a.ctypes.data_as(C.POINTER(C.c_uint64)), n)
    grp = "qkv_attn_o" if ";" not in eng.group_kernels("qkv_attn_o") else "qkv_attn"
    us = eng.time_kernel(grp, 36)
    ctx.sync()
    L.zh_debug_trace_qa(a.ctypes.data_as(C.POINTER(C.c_uint64)), n)
    t = a.reshape(8192, 16)[:256].astype(np.int64)
    base = t[t[:, 0] > 0, 0].min()  # (rows of workgroups that ran)
    print(f"{grp} ({eng.group_kernels(grp)}): {us:.2f} us per launch (events, debug build); "
          "points of the last launch, us from the first workgroup's start / from each workgroup's start:")
    for s, nm in enumerate(QA_POINTS):
        m = t[:, s] > 0
        if not m.any():
            continue
        g, r = (t[m, s] - base) * 0.01, (t[m, s] - t[m, 0]) * 0.01
        print(f"  {nm:24s}: n={m.sum():3d}  abs p50 {np.median(g):6.2f} max {g.max():6.2f}   "
              f"rel min {r.min():6.2f} p50 {np.median(r):6.2f} max {r.max():6.2f}")
        _by_xcd(t, m, g, s)
    eng.deinit()
    ctx.close()


def _by_xcd(t, m, g, s):
    """The per-XCD launches record their XCD (+ 1) in slot 15: abs p50 / max per XCD."""
    xcd = t[:, 15]
    if s > 0 and ((xcd[m] >= 1) & (xcd[m] <= 8)).all():
        per = [(np.median(g[xcd[m] == h + 1]), g[xcd[m] == h + 1].max()) for h in range(8) if (xcd[m] == h + 1).any()]
        print("      by XCD (abs p50/max): " + "  ".join(f"{a:5.2f}/{b:5.2f}" for a, b in per))


RING_POINTS = ["start", "activation landed", "XQ limbs in registers", "ring done", "outputs stored"]


FFN_POINTS = ["start", "activation landed", "XQ limbs in registers", "gate/up done", "down activation in registers",
              "down done", "SwiGLU blocks of the XCD seen", "end", "", "", "", "gate/up tile 0 in LDS"]


MOE_POINTS = ["start", "x, norm, router rows landed", "router logits of the XCD seen", "top-8 selected",
              "gate/up done", "SwiGLU values of the XCD seen", "top-8 ids (polling wave)", "end"]


TILE_POINTS = ["start", "activation staged", "batch 0 in LDS", "batch 1", "batch 2", "batch 3", "batch 4+", "end"]


def ring(group, dump="zh_debug_trace_ring", points=None, moe=False):
    """Per-workgroup timeline of a ring DMMV launch group (zh_ring_q4k.h) or,
    with dump="zh_debug_trace_lpb", of a tile kernel (zh_dmmv_lpb.hip)."""
    points = points or RING_POINTS
    L = hip.lib()
    getattr(L, dump).argtypes = [C.POINTER(C.c_uint64), C.c_uint32]
    ctx = hip.Context(0)
    cfg = dict(MOE_48L if moe else DENSE_8B)
    ctxlen = 8192 if moe else 4096
    cfg["max_ctx"] = ctxlen + 64
    eng = InferenceEngine(ctx, cfg)
    eng.prefill_kv_random(ctxlen, 7)
    eng.generate([17, 18], 2, start_pos=ctxlen)
    ctx.sync()
    n = 8192 * 16
    a = np.zeros(n, np.uint64)
    getattr(L, dump)(a.ctypes.data_as(C.POINTER(C.c_uint64)), n)
    us = eng.time_kernel(group, 36)
    ctx.sync()
    getattr(L, dump)(a.ctypes.data_as(C.POINTER(C.c_uint64)), n)
    t = a.reshape(8192, 16)[:512].astype(np.int64)
    base = t[t[:, 0] > 0, 0].min()  # (rows of workgroups that ran)
    print(f"{group} ({eng.group_kernels(group)}): {us:.2f} us per launch (events, debug build); "
          "points of the last launch, us from the first workgroup's start / from each workgroup's start:")
    for s, nm in enumerate(points):
        m = t[:, s] > 0
        if not m.any():
            continue
        g, r = (t[m, s] - base) * 0.01, (t[m, s] - t[m, 0]) * 0.01
        print(f"  {nm:24s}: n={m.sum():3d}  abs p50 {np.median(g):6.2f} max {g.max():6.2f}   "
              f"rel min {r.min():6.2f} p50 {np.median(r):6.2f} max {r.max():6.2f}")
        _by_xcd(t, m, g, s)
    eng.deinit()
    ctx.close()


def main():
    if not os.environ.get("ZH_LIB_PATH"):
        sys.exit("set ZH_LIB_PATH to the debug build's libzinc_hip.so")
    if "--standalone" in sys.argv[1:]:
        return standalone()
    if "--moe-attn" in sys.argv[1:]:
        return standalone(moe=True)
    if "--qkv-attn" in sys.argv[1:]:
        return qkv_attn(int(sys.argv[sys.argv.index("--ctx") + 1]) if "--ctx" in sys.argv[1:] else 4096)
    if "--ring" in sys.argv[1:]:
        return ring(sys.argv[sys.argv.index("--ring") + 1])
    if "--moe" in sys.argv[1:]:
        return ring("ffn", "zh_debug_trace_moe", MOE_POINTS, moe=True)
    if "--ffn" in sys.argv[1:]:
        return ring("ffn", "zh_debug_trace_ffn", FFN_POINTS)
    if "--tile" in sys.argv[1:]:
        return ring(sys.argv[sys.argv.index("--tile") + 1], "zh_debug_trace_lpb", TILE_POINTS)
    L = hip.lib()
    L.zh_debug_trace_step.argtypes = [C.POINTER(C.c_uint64), C.c_uint32]
    ctx = hip.Context(0)
    cfg = dict(DENSE_8B)
    cfg["max_ctx"] = 4096 + 64
    eng = InferenceEngine(ctx, cfg)
    eng.set_persistent(True)
    eng.prefill_kv_random(4096, 7)
    eng.generate([17, 18], 4, start_pos=4096)
    ctx.sync()
    a = np.zeros(1024 * 32, np.uint64)
    L.zh_debug_trace_step(a.ctypes.data_as(C.POINTER(C.c_uint64)), 1024 * 32)
    t = a.reshape(1024, 32)[:ctx.info()[1]].astype(np.int64)
    base = t[t[:, 0] > 0, 0].min()  # (rows of workgroups that ran)
    names = ["Q/K/V", "attention", "O", "gate/up", "down"]
    print("persistent kernel, layer 10 (us from the first workgroup's start):")
    for s in list(range(10)) + [10]:
        r = (t[:, s] - base) * 0.01
        lab = (names[s // 2] + (" start" if s % 2 == 0 else " end")) if s < 10 else "layer 11 start"
        print(f"  {lab:16s}: min {r.min():7.2f}  p50 {np.median(r):7.2f}  max {r.max():7.2f}")
    print("attention body (last layer of the last step), us from each workgroup's start:")
    print_attn(t[:, 16:])
    eng.deinit()
    ctx.close()


if __name__ == "__main__":
    main()
