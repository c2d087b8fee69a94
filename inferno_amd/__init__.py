"""MI355X-native routed Mixture-of-Experts layer (GGUF K-quant experts).

The compute lives in ``libinferno_moe.so`` (hand-written HIP for gfx950)
behind the C ABI declared in ``include/inferno_moe.h``. This package only
loads that library and offers thin torch-tensor wrappers used by tests and
benchmarks. There is no CPU fallback: if the library is missing, every call
raises.
"""
from ._lib import (  # noqa: F401
    BF16, F32, Q2_K, Q3_K, Q4_K, Q6_K, Q8_0, SCORE_SIGMOID, SCORE_SOFTMAX,
    InfernoError, LayerDesc, lib, lib_path, EXPORTED_SYMBOLS,
)
from . import ops  # noqa: F401
