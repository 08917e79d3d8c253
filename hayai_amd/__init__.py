"""hayai_amd -- MI355X (gfx950) native FFN GEMV engine for Hayai's packed-GGUF hot path.

The product is the C-ABI library ``libhayai_hip.so`` (include/hayai_hip.h) built from
``csrc/``: hand-written HIP kernels for gfx950 plus a C++ runtime over the HIP runtime.
This Python package is the ctypes binding of that ABI plus the seeded synthetic-input
generator used by the tests and the benchmark.  There is no CPU compute path: every
operation runs on the GPU or raises.
"""
from .engine import (  # noqa: F401
    ACT_GELU_TANH,
    ACT_SILU,
    BUF_DEVICE,
    BUF_PINNED_HOST,
    F16,
    F32,
    IQ2_XXS,
    IQ3_XXS,
    Q4_0,
    Q4_K,
    Q6_K,
    Q8_0,
    DeviceBuffer,
    HipEngine,
    HipError,
    LayerPackLayout,
    PendingGemv,
    QuantMatrix,
    StreamingScratch,
    device_count,
    row_bytes,
    validate_gemv_shape,
    validate_gemv_weights,
)
