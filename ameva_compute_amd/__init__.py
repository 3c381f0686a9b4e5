"""ameva MI355X: the quantized ggml backend hot path of ameva-compute (MUL_MAT on Q4_0/Q8_0/Q4_K/Q6_K/I2_S,
RMS_NORM, ROPE, FLASH_ATTN_EXT decode) as hand-written HIP kernels for gfx950 behind a C ABI (include/ameva_hip.h).

Python here is the host mirror over that ABI; torch only provides device memory and streams.
"""
from ._lib import AmevaError, LIB_PATH, lib  # noqa: F401
from . import ops  # noqa: F401
