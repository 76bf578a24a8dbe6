"""CPU-side checks of the C ABI: the library builds/loads and exports every
function include/zinc_hip.h declares, and the Python binding covers them."""
import os
import re
import subprocess

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "zinc_hip.h")
LIB = os.path.join(ROOT, "zinc_amd", "libzinc_hip.so")


def declared_functions():
    src = open(HEADER).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    names = re.findall(r"\b(zh_[a-z0-9_]+)\s*\(", src)
    return sorted(set(names))


def test_header_parses_and_lists_entry_points():
    names = declared_functions()
    assert "zh_dmmv" in names and "zh_engine_generate" in names and len(names) >= 35


def test_library_exports_every_declared_symbol():
    if not os.path.exists(LIB):
        from zinc_amd import build
        build.build(verbose=False)
    out = subprocess.run(["nm", "-D", "--defined-only", LIB], capture_output=True, text=True, check=True).stdout
    exported = set(re.findall(r"\bT (zh_[a-z0-9_]+)", out))
    missing = [n for n in declared_functions() if n not in exported]
    assert not missing, missing


def test_library_loads_and_binding_covers_abi():
    import zinc_amd
    from zinc_amd import hip
    L = zinc_amd.lib()
    for n in declared_functions():
        assert hasattr(L, n)
        assert n in hip.SIGNATURES, f"python binding lacks {n}"
    assert L.zh_status_string(4) == b"ContextLengthExceeded"


def test_no_device_reports_error_not_crash():
    """On a host without a GPU zh_init fails with a status, never falls back."""
    import zinc_amd
    try:
        import torch
        has_gpu = torch.cuda.is_available()
    except Exception:
        has_gpu = False
    if has_gpu:
        return
    import pytest
    with pytest.raises(zinc_amd.ZincError):
        zinc_amd.Context(0)


def test_dmmv_supported_query():
    """zh_dmmv_supported: the counterpart of pipelineForType returning null
    (dmmv.zig:676-690), answered on the host without a device."""
    import zinc_amd
    f = zinc_amd.lib().zh_dmmv_supported
    assert f(12, 4096) == 1 and f(14, 12288) == 1 and f(13, 4096) == 1
    assert f(12, 4000) == 0 and f(14, 128) == 0  # K-quants need whole 256-element super-blocks
    assert f(8, 96) == 1 and f(8, 4096) == 1 and f(8, 100) == 0  # Q8_0: any whole number of 32-blocks
    assert f(39, 2880) == 1 and f(39, 2890) == 0
    assert f(1, 4096) == 0 and f(2, 4096) == 0 and f(0, 4096) == 0  # no DMMV kernel for f16 / f32 / Q4_0
