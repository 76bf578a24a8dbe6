"""GGUF parser robustness: mutated files (truncations, flipped bytes, inflated
counts and lengths) through the parser built for the host with AddressSanitizer
and UndefinedBehaviorSanitizer; every file must be parsed or rejected with an
error, never read out of bounds. The parser is host code, so the sanitizers
apply to exactly the code that reads untrusted bytes."""
import os
import shutil
import struct
import subprocess

import numpy as np
import pytest

from zinc_amd import gguf as G

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)


@pytest.fixture(scope="module")
def driver(tmp_path_factory):
    gxx = shutil.which("g++")
    if gxx is None:
        pytest.skip("no g++")
    out = str(tmp_path_factory.mktemp("fuzz") / "gguf_driver")
    cmd = [gxx, "-std=c++17", "-O1", "-g", "-fsanitize=address,undefined", "-fno-sanitize-recover=all",
           os.path.join(HERE, "fuzz", "gguf_driver.cpp"), os.path.join(ROOT, "zinc_amd", "csrc", "zh_gguf.cpp"),
           "-o", out]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        pytest.skip("sanitizer build unavailable: " + r.stderr[-300:])
    return out


def _seed(path):
    meta = [("general.architecture", "qwen3"), ("qwen3.block_count", (G.U32, 2)),
            ("qwen3.embedding_length", (G.U32, 256)), ("qwen3.attention.head_count", (G.U32, 2)),
            ("qwen3.feed_forward_length", (G.U32, 512)), ("tok", (G.ARRAY, (G.STRING, ["a", "bc", "def"]))),
            ("ids", (G.ARRAY, (G.I32, [1, -2, 3]))), ("f", (G.F64, 2.5))]
    tensors = [("token_embd.weight", [256, 8], 12, np.arange(8 * 144, dtype=np.uint8)),
               ("blk.0.attn_q.weight", [256, 256], 8, np.zeros(256 * 8 * 34, np.uint8)),
               ("n", [256], 0, np.ones(256, np.float32))]
    G.write_gguf(path, meta, tensors)
    return path.read_bytes()


def test_mutated_files_never_read_out_of_bounds(driver, tmp_path):
    raw = _seed(tmp_path / "seed.gguf")
    rng = np.random.default_rng(0)
    files = []
    head_len = raw.index(b"token_embd.weight") + 200  # mutations aimed at the header and tables
    for i in range(400):
        b = bytearray(raw)
        kind = i % 4
        if kind == 0:  # truncate
            b = b[:int(rng.integers(0, len(b)))]
        elif kind == 1:  # flip bytes in the header / tables
            for _ in range(int(rng.integers(1, 8))):
                b[int(rng.integers(0, head_len))] ^= int(rng.integers(1, 256))
        elif kind == 2:  # inflate a length / count field with a huge or edge value
            off = int(rng.integers(0, head_len - 8))
            edge = [2**63, 2**32 + 1, 2**64 - 1, 0xFFFFFFFF, 7]
            b[off:off + 8] = struct.pack("<Q", edge[int(rng.integers(0, len(edge)))])
        else:  # random tag values
            off = int(rng.integers(24, head_len - 4))
            b[off:off + 4] = struct.pack("<I", int(rng.integers(0, 64)))
        p = tmp_path / f"m{i}.gguf"
        p.write_bytes(bytes(b))
        files.append(str(p))
    files.append(str(tmp_path / "seed.gguf"))
    r = subprocess.run([driver] + files, capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stderr[-2000:]
    assert "opened" in r.stdout
