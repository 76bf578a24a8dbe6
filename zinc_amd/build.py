"""Builds libzinc_hip.so (gfx950) in-tree with hipcc.

Usage: python -m zinc_amd.build   (or zinc_amd.build.build())

A debug build (ablation switches read from the environment, per-workgroup
trace points) goes elsewhere and is loaded through ZH_LIB_PATH:
    python -m zinc_amd.build --debug build/debug
and so does a product build with extra defines (A/B of a compile-time variant):
    python -m zinc_amd.build --out build/var/NAME -DNAME=1
"""
import concurrent.futures as cf
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OBJ = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libzinc_hip.so")
SOURCES = ["zh_runtime.hip", "zh_dmmv.hip", "zh_dmmv_lpb.hip", "zh_dmmv_ring.hip", "zh_dmmv_batched.hip", "zh_ops.hip", "zh_engine.hip", "zh_step.hip", "zh_qkv_attn.hip", "zh_ffn_xcd.hip", "zh_moe_xcd.hip", "zh_prefill.hip",
           "zh_gguf.cpp", "zh_sample.hip"]
ARCH = os.environ.get("ZH_OFFLOAD_ARCH", "gfx950")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
FLAGS = [
    "-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}",
    # packed-FP32 instructions stay off (the compiler would otherwise form
    # v_pk_* from float pairs)
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-result", "-Wno-unused-value", "-Wno-unused-command-line-argument", "-Wno-inline-asm",
]


DEBUG_DEFINES = ["-DZH_DEBUG_KNOBS", "-DZH_DEBUG_TRACE"]


def _compile(src, obj_dir=OBJ, defines=()):
    out = os.path.join(obj_dir, os.path.splitext(src)[0] + ".o")
    cmd = [HIPCC, *FLAGS, *defines, "-c", os.path.join(CSRC, src), "-o", out]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{r.stderr}")
    return out


def build(verbose=True, debug_dir=None, out_dir=None, defines=None):
    """debug_dir: the debug build there; out_dir: a product build with extra
    -D defines there (A/B builds of compile-time variants)."""
    alt = debug_dir or out_dir
    obj_dir = os.path.join(alt, "_build") if alt else OBJ
    lib_path = os.path.join(alt, "libzinc_hip.so") if alt else LIB
    defines = DEBUG_DEFINES if debug_dir else list(defines or [])
    os.makedirs(obj_dir, exist_ok=True)
    srcs = [s for s in SOURCES if os.path.exists(os.path.join(CSRC, s))]
    with cf.ThreadPoolExecutor(max_workers=min(len(srcs), 6)) as ex:
        objs = list(ex.map(lambda s: _compile(s, obj_dir, defines), srcs))
    tmp = lib_path + ".tmp"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr}")
    os.replace(tmp, lib_path)
    if verbose:
        print(f"built {lib_path}", file=sys.stderr)
    return lib_path


if __name__ == "__main__":
    if len(sys.argv) == 3 and sys.argv[1] == "--debug":
        build(debug_dir=os.path.abspath(sys.argv[2]))
    elif len(sys.argv) >= 3 and sys.argv[1] == "--out":
        build(out_dir=os.path.abspath(sys.argv[2]), defines=sys.argv[3:])
    else:
        build()
