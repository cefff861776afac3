"""ctypes binding of the C ABI in ``include/eredu_hip.h``.

The shared library is built in-tree by ``eredu_amd.build``.  There is no
fallback: if the library is missing, loading fails with an error that says so.
"""
from __future__ import annotations

import ctypes
import os
import threading

from .build import LIB_PATH

EQ_DTYPE_F32, EQ_DTYPE_F16, EQ_DTYPE_BF16, EQ_DTYPE_U8 = 0, 1, 2, 3
EQ_ENDIAN_LITTLE, EQ_ENDIAN_BIG = 0, 1
EQ_DEQUANT_AFFINE, EQ_DEQUANT_NATIVE = 0, 1

# Every exported entry point with its ctypes signature (mirrors include/eredu_hip.h).
_vp, _i64, _i32, _b = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_bool
SIGNATURES = {
    "eq_last_error": ([], ctypes.c_char_p),
    "eq_version": ([], _i32),
    "eq_quantized_matmul": ([_vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _b, _i32, _i32, ctypes.c_char_p, _i32, _i32, _vp], _i32),
    "eq_dequantize": ([_vp, _vp, _vp, _vp, _i64, _i64, _i32, _i32, ctypes.c_char_p, _i32, _i32, _vp], _i32),
    "eq_gguf_convert_affine": ([_vp, _vp, _vp, _vp, _i64, _i32, _i64, _i64, _i32, _vp], _i32),
    "eq_gguf_convert_mxfp4": ([_vp, _vp, _vp, _i64, _i64, _i64, _vp], _i32),
    "eq_gguf_dequantize": ([_vp, _vp, _i64, _i32, _i64, _i64, _i32, _i32, _i32, _vp], _i32),
    "eq_gguf_linear": ([_vp, _vp, _vp, _i64, _i32, _i64, _i64, _i64, _i32, _i32, _vp], _i32),
    "eq_gguf_embedding": ([_vp, _vp, _i64, _i32, _i64, _i64, _vp, _i64, _i32, _i32, _vp], _i32),
    "eq_gguf_grouped_linear": ([_vp, _vp, _vp, _i64, _i32, _i64, _i64, _i64, _vp, _i64, _i32, _i32, _b, _vp], _i32),
    "eq_gather_qmm": ([_vp, _vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _i64, _b, _i32, _i32,
                       ctypes.c_char_p, _i32, _i32, _b, _vp], _i32),
    "eq_quantize": ([_vp, _vp, _vp, _vp, _i64, _i64, _i32, _i32, ctypes.c_char_p, _i32, _vp], _i32),
    "eq_rms_norm": ([_vp, _vp, _vp, _vp, _i64, _i64, ctypes.c_float, _i32, _vp], _i32),
    "eq_rope_attention_decode": ([_vp, _vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i32, _i32, _i32, ctypes.c_float,
                                  _i32, _vp], _i32),
    "eq_rope_attention_decode_noalloc": ([_vp, _vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i32, _i32, _i32,
                                          ctypes.c_float, _i32, _vp], _i32),
    "eq_rope_attention_decode_at": ([_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i64, _i32, _i32, _i32,
                                     ctypes.c_float, _i32, _vp], _i32),
    "eq_advance_position": ([_vp, _vp], _i32),
    "eq_silu_mul": ([_vp, _vp, _vp, _i64, _i32, _vp], _i32),
    "eq_embedding": ([_vp, _vp, _vp, _i64, _i64, _i64, _i32, _vp], _i32),
    "eq_argmax": ([_vp, _vp, _i64, _i64, _i32, _vp], _i32),
}



class QmmProblem(ctypes.Structure):
    """eq_qmm_problem of include/eredu_hip.h."""

    _fields_ = [("y", _vp), ("x", _vp), ("w", _vp), ("scales", _vp), ("biases", _vp), ("N", _i64), ("K", _i64)]


SIGNATURES["eq_quantized_matmul_batched"] = (
    [ctypes.POINTER(QmmProblem), _i32, _i64, _b, _i32, _i32, ctypes.c_char_p, _i32, _i32, _vp], _i32)

EQ_PROLOGUE_SILU_MUL, EQ_PROLOGUE_RMS_NORM = 1, 2


class ActivationPrologue(ctypes.Structure):
    """eq_activation_prologue of include/eredu_hip.h."""

    _fields_ = [("kind", _i32), ("second", _vp), ("weight", _vp), ("hidden_out", _vp), ("eps", ctypes.c_float)]


SIGNATURES["eq_quantized_matmul_batched_prologue"] = (
    [ctypes.POINTER(QmmProblem), _i32, _i64, _b, _i32, _i32, ctypes.c_char_p, _i32, _i32,
     ctypes.POINTER(ActivationPrologue), _vp], _i32)
SIGNATURES["eq_quantized_matmul_swiglu"] = (
    [_vp, _vp, _vp, _vp, _vp, _i64, _i64, _i32, _i32, ctypes.c_char_p, _i32, _i32, ctypes.POINTER(ActivationPrologue),
     _vp], _i32)

_lib = None
_lock = threading.Lock()


class EreduError(RuntimeError):
    """Error raised when a library call fails (the reference's Exception{what})."""


def lib() -> ctypes.CDLL:
    """The HIP library: eredu_amd/_lib/liberedu_hip.so, or the file the
    EREDU_AMD_LIB environment variable names (another build of it, e.g. the
    sanitizer build of the host code that tests/test_host_sanitize.py makes)."""
    global _lib
    with _lock:
        if _lib is None:
            path = os.environ.get("EREDU_AMD_LIB") or LIB_PATH
            if not os.path.exists(path):
                raise EreduError(
                    f"HIP kernel library not found at {path}; build it with `python -m eredu_amd.build`"
                )
            L = ctypes.CDLL(path)
            for name, (args, res) in SIGNATURES.items():
                fn = getattr(L, name)
                fn.argtypes = args
                fn.restype = res
            _lib = L
    return _lib


def check(status: int) -> None:
    if status != 0:
        msg = lib().eq_last_error().decode("utf-8", "replace")
        raise EreduError(msg or "unknown error")
