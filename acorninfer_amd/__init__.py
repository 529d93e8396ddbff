"""acorninfer_amd: MI355X (gfx950) HIP implementation of AcornInfer's Qwen3
decode hot path behind the reference's `acorninfer/ops` + `acorninfer/quant`
Python call signatures and its paged-KV block-table layout.

Kernels live in libacorn_hip.so (acorninfer_amd/csrc, C-ABI in
include/acorn_hip.h), loaded through ctypes by acorninfer_amd._lib.
"""

__version__ = "0.1.0"
