"""MI355X (gfx950) implementation of RapidOCRvl's ERNIE text-decoder step.

The compute lives in libpocr_hip.so (rapidocrvl_amd/csrc, C ABI in
include/pocr_hip.h); this package is its ctypes binding plus the seeded
synthetic inputs used by the tests and benchmarks.
"""
from .config import ERNIE_0P3B, DecoderConfig  # noqa: F401
from .lib import (Context, Model, PocrError, QMatrix, Sequence, device_count, load, mm_positions,  # noqa: F401
                  quantize_rows, unpack_rows)
