"""ctypes binding of libh3fp8.so (the C ABI declared in include/h3fp8.h).

The library is built in-tree (``minimax-h3-2x-dgx-spark-tp2_amd/build.py``) next to this file.  There is no fallback:
if the library is missing or fails to load, every call raises -- the product path runs the HIP kernels or nothing.
"""
from __future__ import annotations

import ctypes
import os
import threading

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libh3fp8.so")
ABI_VERSION = 1

H3FP8_DT_BF16 = 0
H3FP8_DT_FP16 = 1
H3FP8_DT_F32 = 2
MAX_GROUPS = 8
NOALLOC_MAX_ROWS = 262144       # H3FP8_NOALLOC_MAX_ROWS

_lib = None
_lock = threading.Lock()

P = ctypes.c_void_p
I64 = ctypes.c_int64
I = ctypes.c_int


class Group(ctypes.Structure):
    """``h3fp8_group`` of include/h3fp8.h."""
    _fields_ = [("a", P), ("lda", I64), ("w", P), ("ldw", I64), ("sa", P), ("sa_stride", I64), ("sb", P),
                ("sb_stride", I64), ("y", P), ("ldy", I64), ("M", I64), ("N", I64), ("K", I64)]


_SIGS = {
    "h3fp8_abi_version": ([], I),
    "h3fp8_last_error": ([], ctypes.c_char_p),
    "h3fp8_init": ([], I),
    "h3fp8_quant_rows": ([P, I64, I64, I64, P, I64, P, P], I),
    "h3fp8_quant_rows_amax": ([P, I64, I64, I64, P, P, I64, P, P], I),
    "h3fp8_quant_segments": ([P, I64, I64, I64, I64, I64, P, I64, P, P], I),
    "h3fp8_gemm": ([P, I64, P, I64, P, I64, P, I64, P, P, I64, I, I64, I64, I64, P, P], I),
    "h3fp8_gemm_quant": ([P, I64, P, I64, P, I64, P, I64, P, P, I64, I64, I64, I64, P, P, I64, P, P], I),
    "h3fp8_gemm_quant_noalloc": ([P, I64, P, I64, P, I64, P, I64, P, P, I64, I64, I64, I64, P, I64, P, P], I),
    "h3fp8_gemm_swiglu": ([P, I64, P, I64, P, I64, P, I64, P, P, I64, P, I64, I64, I64, P], I),
    "h3fp8_gemm_swiglu_quant": ([P, I64, P, I64, P, I64, P, I64, P, I64, I64, I64, P, P, P, I64, P, P], I),
    "h3fp8_scale_swiglu": ([P, I64, P, I64, P, I64, P, I64, I64, P, I64, P], I),
    "h3fp8_scale_swiglu_quant": ([P, I64, P, I64, P, I64, P, I64, I64, P, I64, P, P], I),
    "h3fp8_silu_mul_quant": ([P, I64, I64, I64, P, I64, P, P], I),
    "h3fp8_rms_quant": ([P, I64, P, P, I64, P, I64, I64, P, I64, I, I64, I64, ctypes.c_float, P, I64, P, P, I64, P],
                        I),
    "h3fp8_gate_rms_quant": ([P, I64, P, I64, P, I64, P, P, I64, P, I64, I64, P, I64, I, I64, I64, ctypes.c_float,
                              P, I64, P, I64, P, P, I64, P], I),
    "h3fp8_scale_gate_rms_quant": ([P, I64, P, P, P, P, I64, P, I64, P, P, I64, P, I64, I64, P, I64, I, I64, I64,
                                    ctypes.c_float, P, I64, P, I64, P, P, I64, P], I),
    "h3fp8_scale_indexed_gate": ([P, I64, P, P, P, P, I64, P, I64, I64, P, I64, I, I64, I64, P, I64, P], I),
    "h3fp8_scale_qk_norm_rope": ([P, I64, P, P, P, I64, I, I, P, P, P, I64, I, ctypes.c_float, P, I64, I64, P, I64,
                                  I64, P], I),
    "h3fp8_scale_qkv_norm_rope": ([P, I64, P, P, P, I64, I, I, I, P, P, P, I64, I, ctypes.c_float, P, I64, I64, P,
                                   I64, I64, P, I64, I64, P], I),
    "h3fp8_scale_bias_cast": ([P, I64, P, I64, P, I64, P, P, I64, I, I64, I64, P], I),
    "h3fp8_grouped_gemm": ([ctypes.POINTER(Group), I, P], I),
    "h3fp8_selfcheck_e4m3": ([ctypes.POINTER(ctypes.c_uint64), ctypes.POINTER(ctypes.c_uint64)], I),
    "h3fp8_selfcheck_bf16": ([ctypes.POINTER(ctypes.c_uint64), ctypes.POINTER(ctypes.c_uint64)], I),
    "h3fp8_copy_silu_table": ([P, P], I),
    "h3fp8_mfma_loop": ([P, I64, I64, ctypes.c_uint32, P], I),
}

EXPORTS = tuple(_SIGS)


class H3Fp8Error(RuntimeError):
    """A non-zero status from the C ABI (message from h3fp8_last_error)."""

    def __init__(self, fn: str, rc: int, msg: str):
        super().__init__(f"{fn} returned {rc}: {msg}")
        self.fn, self.rc = fn, rc


def load(path: str | None = None) -> ctypes.CDLL:
    """Load (once) and type the library; raises if it is missing or its ABI version differs."""
    global _lib
    if _lib is not None and path is None:
        return _lib
    with _lock:
        if _lib is not None and path is None:
            return _lib
        p = path or LIB_PATH
        if not os.path.exists(p):
            raise FileNotFoundError(
                f"{p} is missing: build it with `python minimax-h3-2x-dgx-spark-tp2_amd/build.py` "
                "(the online-FP8 path has no fallback)")
        L = ctypes.CDLL(p)
        for name, (args, res) in _SIGS.items():
            f = getattr(L, name)
            f.argtypes = args
            f.restype = res
        v = L.h3fp8_abi_version()
        if v != ABI_VERSION:
            raise RuntimeError(f"libh3fp8 ABI version {v}, expected {ABI_VERSION}")
        if path is None:
            _lib = L
        return L


def call(name: str, *args) -> None:
    """Call an entry point and raise H3Fp8Error on a non-zero status."""
    L = load()
    rc = getattr(L, name)(*args)
    if rc != 0:
        msg = L.h3fp8_last_error()
        raise H3Fp8Error(name, rc, msg.decode() if msg else "")
