"""tcb_amd -- MI355X (gfx950) implementation of TR's quantized GGUF matmul.

The product is libtrhip.so (HIP kernels behind the C-ABI in include/trhip.h). This package holds its
ctypes binding (_lib), a host mirror of the reference's operator interface (backend), synthetic-input
generators and GGUF encoders (synth) and the build script (build).
"""
from ._lib import Q8, Q4, Q4K, Q6K, MODE_EXACT, MODE_FAST, F32, F16, BF16  # noqa: F401
from .backend import (  # noqa: F401
    BLOCK, NAMES, CheckQuantScales, Context, DeviceBuffer, QuantBackend, QuantWeight, TrhipError, device_count,
)
