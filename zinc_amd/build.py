"""Builds libzinc_hip.so (gfx950) in-tree with hipcc.

Usage: python -m zinc_amd.build   (or zinc_amd.build.build())

A debug build (ablation switches read from the environment, per-workgroup
trace points) goes elsewhere and is loaded through ZH_LIB_PATH:
    python -m zinc_amd.build --debug OUT_DIR
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


def build(verbose=True, debug_dir=None):
    obj_dir = os.path.join(debug_dir, "_build") if debug_dir else OBJ
    lib_path = os.path.join(debug_dir, "libzinc_hip.so") if debug_dir else LIB
    defines = DEBUG_DEFINES if debug_dir else []
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
    else:
        build()
