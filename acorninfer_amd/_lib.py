"""ctypes binding of libacorn_hip.so (the C-ABI in include/acorn_hip.h).

torch is imported first so that the library's libamdhip64.so.7 dependency
resolves to the HIP runtime torch already loaded: kernels launched here and
torch's own work share one runtime, one set of streams and one hipGraph
capture.

There is no fallback: if the library has not been built, or a call is made
with CPU tensors, the operator raises.
"""
from __future__ import annotations

import ctypes
import os
from pathlib import Path

import torch

LIB_PATH = Path(os.environ.get(
    "ACORN_HIP_LIB", Path(__file__).resolve().parent / "_lib" / "libacorn_hip.so"))

# dtype / format codes (acorn_hip.h)
F32, F16, BF16 = 0, 1, 2
WFMT_BF16, WFMT_W8, WFMT_W4, WFMT_F32, WFMT_W4B, WFMT_W8B, WFMT_BF16B = 0, 1, 2, 3, 4, 5, 6

OK = 0
ERR_SHAPE, ERR_DTYPE, ERR_VALUE, ERR_UNSUPPORTED, ERR_SCRATCH, ERR_HIP = -1, -2, -3, -4, -5, -1000
K3_SCRATCH_BYTES = 32 << 20     # ACORN_K3_SCRATCH_BYTES

_DTYPE_CODE = {torch.float32: F32, torch.float16: F16, torch.bfloat16: BF16}

_vp = ctypes.c_void_p
_i64 = ctypes.c_int64
_i32 = ctypes.c_int
_f32 = ctypes.c_float
_pi = ctypes.POINTER(ctypes.c_int)

# name -> argtypes (restype is int for all)
_SIGNATURES = {
    "acorn_version": [],
    "acorn_fused_add_rmsnorm": [_vp, _vp, _vp, _vp, _vp, _i64, _i64, _f32, _i32, _i32, _vp],
    "acorn_fused_add_rmsnorm_partials": [_vp, _i64, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _f32,
                                         _i32, _i32, _vp],
    "acorn_rope_inplace": [_vp, _i64, _i64, _i64, _vp, _i32, _vp, _i32, _vp],
    "acorn_qknorm_rope_inplace": [_vp, _vp, _i64, _i64, _i64, _i64, _vp, _vp, _f32, _vp, _i32,
                                  _vp, _i32, _i32, _vp],
    "acorn_qkv_epilogue": [_vp, _i64, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64,
                           _i64, _vp, _vp, _f32, _vp, _vp, _i32, _i32, _vp],
    "acorn_paged_attention": [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64,
                              _i64, _i64, _i64, _i64, _f32, _i32, _vp],
    "acorn_paged_attention_noalloc": [_vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64,
                                      _i64, _i64, _i64, _i64, _f32, _i32, _vp],
    "acorn_paged_prefill_attention": [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64,
                                      _i64, _i64, _i64, _i64, _i64, _i64, _f32, _i32, _vp],
    "acorn_paged_attention_qkv": [_vp, _i64, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp,
                                  _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _f32,
                                  _vp, _vp, _f32, _vp, _vp, _i32, _i32, _vp],
    "acorn_paged_attention_qkv_supported": [_i64, _i64, _i64, _i64, _i64, _i64, _i32, _i32],
    "acorn_quant_gemm": [_vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i32, _vp, _vp],
    "acorn_splitk_reduce": [_vp, _i64, _i64, _vp, _i32, _vp],
    "acorn_dequant_w4b": [_vp, _vp, _vp, _i64, _i64, _vp],
    "acorn_gemm_plan": [_i64, _i64, _i64, _i32, _vp],
    "acorn_quant_gemm_swiglu": [_vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i32, _vp, _vp],
    "acorn_gemm_swiglu_plan": [_i64, _i64, _i64, _i32, _vp],
    "acorn_quant_gemm_norm": [_vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i32, _vp, _i32, _vp,
                              _f32, _vp, _vp, _vp, _vp, _vp, _vp],
    "acorn_embedding": [_vp, _vp, _vp, _i64, _i64, _i64, _i32, _vp],
    "acorn_silu_mul": [_vp, _i64, _vp, _vp, _i64, _i64, _i32, _i32, _vp],
    "acorn_argmax": [_vp, _i64, _i64, _vp, _i32, _vp],
    "acorn_sample": [_vp, _i64, _i64, _i32, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp],
    "acorn_kv_scatter": [_vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _i32,
                         _vp],
}

_lib = None


class AcornError(RuntimeError):
    """A launch failure reported by the HIP runtime."""


def lib() -> ctypes.CDLL:
    """Load (once) and return the library; raise if it was never built."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"libacorn_hip.so not found at {LIB_PATH}; build it with "
                "`python -m acorninfer_amd.build` (no fallback path exists)")
        handle = ctypes.CDLL(str(LIB_PATH))
        for name, args in _SIGNATURES.items():
            fn = getattr(handle, name)
            fn.argtypes = args
            fn.restype = ctypes.c_int
        _lib = handle
    return _lib


def exported_symbols() -> list[str]:
    return list(_SIGNATURES)


def check(rc: int, op: str) -> None:
    """Map a C-ABI return code to the exception the reference raises."""
    if rc == OK:
        return
    if rc == ERR_SHAPE:
        raise AssertionError(f"{op}: shape/contiguity contract violated")
    if rc == ERR_DTYPE:
        raise ValueError(f"{op}: unsupported dtype")
    if rc == ERR_VALUE:
        raise ValueError(f"{op}: bad argument")
    if rc == ERR_SCRATCH:
        raise ValueError(f"{op}: the request needs more than the {K3_SCRATCH_BYTES >> 20} MiB "
                         "of fixed device scratch of the allocation-free entry point")
    if rc == ERR_UNSUPPORTED:
        raise NotImplementedError(f"{op}: configuration not supported by the HIP kernels")
    if rc <= ERR_HIP:
        raise AcornError(f"{op}: HIP error {ERR_HIP - rc}")
    raise AcornError(f"{op}: error {rc}")


def dtype_code(t: torch.Tensor) -> int:
    try:
        return _DTYPE_CODE[t.dtype]
    except KeyError:
        raise ValueError(f"unsupported dtype {t.dtype}") from None


def stream_ptr(device: torch.device | None = None) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def require_gpu(*tensors: torch.Tensor | None) -> None:
    for t in tensors:
        if t is not None and t.device.type != "cuda":
            raise ValueError(
                f"acorninfer_amd operators run only on the GPU (got a {t.device} tensor)")
