"""zinc_amd — MI355X (gfx950) HIP backend for ZINC's per-token decode loop.

The compute path is libzinc_hip.so (hand-written HIP kernels behind the C ABI
in include/zinc_hip.h). This package is the Python binding and the
InferenceEngine mirror; it has no CPU fallback.
"""
from .hip import (F16, F32, MXFP4, Q4_K, Q5_K, Q6_K, Q8_0, Buffer, Context, SamplingParams, ZincError,  # noqa: F401
                  lib, tensor_bytes)
from .engine import DENSE_8B, MOE_48L, DecodeState, InferenceEngine, KvPagePool  # noqa: F401
