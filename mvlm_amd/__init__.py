"""MI355X (gfx950) HIP implementation of MVLM's matmul hot path.

The compute lives in libmvlm_hip.so (C ABI: include/mvlm_hip.h); `native`
binds it with ctypes, and `engine/` holds the C++ drop-in for the reference's
mgpu::dispatch_* / create_weight_image / BufferPool interface.
"""
from .native import (BF16, F16, F32, LAYOUT_KN, LAYOUT_NK, Q4_0, Q8_0, Buffer, Device, Event, Gguf,  # noqa: F401
                     MvlmError, Plan, Weight, device_count, ggml_type_size, lib)
