"""CPU oracle of the online-FP8 linear path -- TEST INFRASTRUCTURE ONLY.

Python face of ``oracle.c`` (built by ``make -C oracle`` into ``liboracle.so``) plus the fp32 matmul in numpy.  Only
``tests/``, ``__graft_entry__.smoke()`` and the CPU-baseline leg of ``bench.py`` may import this module, and only to
check or to time the reference algorithm; the product path never calls it.

Each function names the reference code it restates (paths relative to the reference checkout):

* ``quant_rows``          h3_tp2/fp8_quant_fuse.py:302-307 (``quant_torch``), formula at :11-13, helpers :92-121
* ``e4m3fn_from_f32``     the ``.to(torch.float8_e4m3fn)`` cast of fp8_quant_fuse.py:306
* ``bf16_rne``            h3_tp2/fp8_swiglu.py:38-45 (``_round_bf16``) and torch's fp32 -> bf16 cast
* ``epilogue``            h3_tp2/fp8_gemm.py:37-54, :120-126, :174-185 (``sb * acc`` first, then ``sa``; bias by fma)
* ``silu_table``          h3_tp2/fp8_swiglu.py:69, :211 (``bf16(g / (1 + exp(-g)))``, exp correctly rounded here)
* ``swiglu_bf16``         h3_tp2/fp8_swiglu.py:64-70, :210-212; fp8_quant_fuse.py:262-278 (before its quant)
* ``scale_swiglu``        h3_tp2/fp8_swiglu.py:47-70, :203-212
* ``scale_swiglu_quant``  h3_tp2/fp8_swiglu.py:72-103
* ``dequant_matmul``      h3_tp2/fp8_consumers.py:518-523 (``a.float() @ w.float().t()``, fp32); ``matmul_f32`` is the
                          same product through numpy's BLAS (any summation order) for large shapes.
* ``rms_quant``           h3_tp2/fp8_quant_fuse.py:143-188, :330-346: the stock ``rms_norm_indexed_scale_shift`` as
                          tests/fake_h3_consumers.py:77-84 states it, then ``quant_rows``
* ``gate_rms_quant``      h3_tp2/fp8_quant_fuse.py:191-243, :349-369: ``indexed_gate_rms_norm_scale_shift``
                          (tests/fake_h3_consumers.py:66-74), then ``quant_rows``
* ``row_sumsq``           the sum of squares of those producers, in fp64, in the HIP kernel's fixed order
* ``qk_norm_rope``        the stock ``fused_qk_norm_rope`` half-split kernel as tests/fake_h3_consumers.py:29-48 states
                          it (head_dim 128, rotary 96); the fused consumer of h3_tp2/fp8_consumers.py:131-193 is
                          ``epilogue`` (the scale pass) followed by it

Pinning (what each function is checked against, in tests/test_oracle.py): the e4m3fn/bf16/fp16 casts against torch's
and numpy's own casts on exhaustive or dense sweeps; ``quant_rows`` against known answers of the reference's tests
(zero row -> MIN_SCALE, every positive finite bf16 as a row maximum against IEEE division done by numpy), against the
e4m3 grid (every code re-quantises to itself) and against brute-force nearest-grid search; ``epilogue`` against the
order-sensitive known answer of tests/test_fp8_gemm.py:67-75 and against float64 arithmetic; ``silu_table`` against
torch's CPU exp on all 65536 bf16 inputs and against float64; ``dequant_matmul`` against exact integer products;
``row_sumsq`` against the exact sum (``math.fsum``); ``rms_quant`` / ``gate_rms_quant`` against closed forms
(constant rows, power-of-two scale invariance), an index permutation, torch's CPU evaluation of the stand-ins (equal
residual, modulated rows within one bf16 ulp) and their own composition with ``quant_rows``.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib = None

FP8_MAX = 448.0
MIN_SCALE = np.float32(1.0 / (448.0 * 512.0))


def build(force: bool = False) -> str:
    """Compile ``oracle.c`` with the committed Makefile (gcc); returns the library path."""
    src = os.path.join(_HERE, "oracle.c")
    if force or not os.path.exists(_LIB_PATH) or os.path.getmtime(_LIB_PATH) < os.path.getmtime(src):
        subprocess.run(["make", "-s", "-C", _HERE, "-B", "liboracle.so"], check=True)
    return _LIB_PATH


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        P, I64, I = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int
        L.oracle_quant_rows.argtypes = [P, I64, I64, I64, P, I64, P]
        L.oracle_epilogue.argtypes = [P, I64, I64, P, P, P, I, P]
        L.oracle_silu_table.argtypes = [P]
        L.oracle_swiglu_bf16.argtypes = [P, I64, I64, I64, P]
        L.oracle_scale_swiglu.argtypes = [P, I64, I64, P, P, P, P]
        L.oracle_scale_swiglu_quant.argtypes = [P, I64, I64, P, P, P, P, P]
        L.oracle_dequant_matmul.argtypes = [P, I64, P, I64, I64, I64, I64, P]
        L.oracle_row_sumsq.argtypes = [P, I64]
        L.oracle_row_sumsq.restype = ctypes.c_double
        F = ctypes.c_float
        L.oracle_rms_quant.argtypes = [P, I64, P, P, I64, P, I64, P, I64, I64, F, P, P, P]
        L.oracle_gate_rms_quant.argtypes = [P, I64, P, I64, P, I64, P, P, I64, P, I64, P, I64, I64, F, P, P, P, P]
        L.oracle_qk_norm_rope.argtypes = [P, I64, I64, P, P, F, P]
        L.oracle_e4m3fn_from_f32.argtypes = [ctypes.c_float]
        L.oracle_e4m3fn_from_f32.restype = ctypes.c_uint8
        L.oracle_bf16_rne.argtypes = [ctypes.c_float]
        L.oracle_bf16_rne.restype = ctypes.c_uint16
        L.oracle_min_scale.restype = ctypes.c_float
        for name in ("oracle_e4m3fn_from_f32_array", "oracle_bf16_rne_array", "oracle_fp16_rne_array"):
            getattr(L, name).argtypes = [P, I64, P]
        _lib = L
    return _lib


def _p(a: np.ndarray) -> int:
    assert a.flags["C_CONTIGUOUS"], "oracle arrays must be C-contiguous"
    return a.ctypes.data


def _u16(a) -> np.ndarray:
    a = np.ascontiguousarray(a)
    return a.view(np.uint16) if a.dtype.itemsize == 2 else a.astype(np.uint16)


def bf16_bits_from_f32(x: np.ndarray) -> np.ndarray:
    """Vectorised fp32 -> bf16 RNE bits (same rule as oracle_bf16_rne, NaN quietened)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    r[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
    return r


def bf16_to_f32(bits: np.ndarray) -> np.ndarray:
    return (np.ascontiguousarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def e4m3_to_f32(codes: np.ndarray) -> np.ndarray:
    """Decode e4m3fn codes (uint8) to fp32 through a 256-entry table."""
    return _E4M3_LUT()[np.asarray(codes, dtype=np.uint8)]


_lut_cache: dict = {}


def _E4M3_LUT() -> np.ndarray:
    t = _lut_cache.get("e4m3")
    if t is None:
        f = lib().oracle_e4m3fn_to_f32
        f.argtypes = [ctypes.c_uint8]
        f.restype = ctypes.c_float
        t = np.array([f(i) for i in range(256)], dtype=np.float32)
        _lut_cache["e4m3"] = t
    return t


def e4m3fn_from_f32(x: np.ndarray) -> np.ndarray:
    """Elementwise (shape kept) fp32 -> e4m3fn (RNE) through the C routine (the ``.to(float8_e4m3fn)`` of the reference)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    shape = x.shape
    x = x.ravel()
    out = np.empty(x.size, dtype=np.uint8)
    lib().oracle_e4m3fn_from_f32_array(_p(x), x.size, _p(out))
    return out.reshape(shape)


def bf16_rne(x: np.ndarray) -> np.ndarray:
    """Elementwise (shape kept) fp32 -> bf16 bits through the C routine (``_round_bf16`` / torch's cast)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    shape = x.shape
    x = x.ravel()
    out = np.empty(x.size, dtype=np.uint16)
    lib().oracle_bf16_rne_array(_p(x), x.size, _p(out))
    return out.reshape(shape)


def fp16_rne(x: np.ndarray) -> np.ndarray:
    """Elementwise (shape kept) fp32 -> fp16 bits through the C routine (torch's ``.to(torch.float16)``)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    shape = x.shape
    x = x.ravel()
    out = np.empty(x.size, dtype=np.uint16)
    lib().oracle_fp16_rne_array(_p(x), x.size, _p(out))
    return out.reshape(shape)


def quant_rows(x_bf16_bits: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """bf16 [M, K] (uint16 bit patterns) -> (e4m3fn codes uint8 [M, K], fp32 scale [M])."""
    x = _u16(x_bf16_bits)
    M, K = x.shape
    q = np.empty((M, K), dtype=np.uint8)
    s = np.empty((M,), dtype=np.float32)
    lib().oracle_quant_rows(_p(x), M, K, K, _p(q), K, _p(s))
    return q, s


def epilogue(acc: np.ndarray, sa: np.ndarray, sb: np.ndarray, bias_bits: np.ndarray | None = None,
             out_fp16: bool = False) -> np.ndarray:
    """fp32 [M, N] accumulator -> bf16 (or fp16) bit patterns [M, N]: round(sa[m] * (sb[n] * acc)), bias by fma."""
    acc = np.ascontiguousarray(acc, dtype=np.float32)
    M, N = acc.shape
    sa = np.ascontiguousarray(np.broadcast_to(np.asarray(sa, np.float32).reshape(-1), (M,)))
    sb = np.ascontiguousarray(np.broadcast_to(np.asarray(sb, np.float32).reshape(-1), (N,)))
    b = None if bias_bits is None else _u16(bias_bits)
    y = np.empty((M, N), dtype=np.uint16)
    lib().oracle_epilogue(_p(acc), M, N, _p(sa), _p(sb), None if b is None else _p(b), int(out_fp16), _p(y))
    return y


def silu_table() -> np.ndarray:
    """bf16 bits g -> bf16 bits of silu(g) rounded to bf16, for all 65536 inputs."""
    t = _lut_cache.get("silu")
    if t is None:
        t = np.empty(65536, dtype=np.uint16)
        lib().oracle_silu_table(_p(t))
        _lut_cache["silu"] = t
    return t


def swiglu_bf16(gu_bits: np.ndarray) -> np.ndarray:
    """bf16 [M, 2F] = [gate | up] -> bf16 h [M, F] (bit patterns)."""
    gu = _u16(gu_bits)
    M, W = gu.shape
    F = W // 2
    h = np.empty((M, F), dtype=np.uint16)
    lib().oracle_swiglu_bf16(_p(gu), M, F, W, _p(h))
    return h


def scale_swiglu(acc: np.ndarray, sa: np.ndarray, sb: np.ndarray, bias_bits: np.ndarray | None = None) -> np.ndarray:
    acc = np.ascontiguousarray(acc, dtype=np.float32)
    M, W = acc.shape
    F = W // 2
    sa = np.ascontiguousarray(sa, dtype=np.float32).reshape(-1)
    sb = np.ascontiguousarray(sb, dtype=np.float32).reshape(-1)
    b = None if bias_bits is None else _u16(bias_bits)
    h = np.empty((M, F), dtype=np.uint16)
    lib().oracle_scale_swiglu(_p(acc), M, F, _p(sa), _p(sb), None if b is None else _p(b), _p(h))
    return h


def scale_swiglu_quant(acc: np.ndarray, sa: np.ndarray, sb: np.ndarray, bias_bits: np.ndarray | None = None):
    acc = np.ascontiguousarray(acc, dtype=np.float32)
    M, W = acc.shape
    F = W // 2
    sa = np.ascontiguousarray(sa, dtype=np.float32).reshape(-1)
    sb = np.ascontiguousarray(sb, dtype=np.float32).reshape(-1)
    b = None if bias_bits is None else _u16(bias_bits)
    q = np.empty((M, F), dtype=np.uint8)
    s = np.empty((M,), dtype=np.float32)
    lib().oracle_scale_swiglu_quant(_p(acc), M, F, _p(sa), _p(sb), None if b is None else _p(b), _p(q), _p(s))
    return q, s


def dequant_matmul(a_codes: np.ndarray, w_codes: np.ndarray) -> np.ndarray:
    """fp32 acc[m, n] = sum_k a[m, k] * w[n, k] (K ascending, C loop; small shapes)."""
    a = np.ascontiguousarray(a_codes, dtype=np.uint8)
    w = np.ascontiguousarray(w_codes, dtype=np.uint8)
    M, K = a.shape
    N = w.shape[0]
    acc = np.empty((M, N), dtype=np.float32)
    lib().oracle_dequant_matmul(_p(a), K, _p(w), K, M, N, K, _p(acc))
    return acc


def matmul_f32(a_codes: np.ndarray, w_codes: np.ndarray) -> np.ndarray:
    """The same fp32 product through numpy's BLAS (multithreaded, any summation order): large shapes."""
    lut = _E4M3_LUT()
    return lut[a_codes] @ lut[w_codes].T


def linear(x_bf16_bits: np.ndarray, w_codes: np.ndarray, sb: np.ndarray, bias_bits=None, out_fp16=False):
    """The whole reference CPU path of one online-FP8 linear: per-token quant of X, fp32 product, epilogue."""
    q, sa = quant_rows(x_bf16_bits)
    return epilogue(matmul_f32(q, w_codes), sa, sb, bias_bits, out_fp16), q, sa


def row_sumsq(x_bf16_bits: np.ndarray) -> float:
    """sum_k fp32(x_k * x_k) of one bf16 row (H % 8 == 0), in fp64, in the HIP kernel's fixed order."""
    x = bf16_to_f32(_u16(x_bf16_bits).reshape(-1))
    x = np.ascontiguousarray(x, dtype=np.float32)
    return float(lib().oracle_row_sumsq(_p(x), x.size))


def _table(t: np.ndarray) -> tuple[np.ndarray, int]:
    """A [B, H] bf16 table (bit patterns, any row stride) -> (contiguous-row array, row stride in elements)."""
    t = _u16(t)
    return t, t.shape[1]


def rms_quant(x_bits, weight_bits, shift_bits, scale_bits, indices, eps: float):
    """bf16 x [M, H], weight [H], shift / scale [B, H] tables, indices [M] ->
    (h bf16 bits [M, H], fp8 codes [M, H], fp32 scale [M])."""
    x = _u16(x_bits)
    M, H = x.shape
    w = _u16(weight_bits).reshape(-1)
    sh, ldsh = _table(shift_bits)
    sc, ldsc = _table(scale_bits)
    idx = np.ascontiguousarray(np.asarray(indices).reshape(-1), dtype=np.int64)
    assert idx.size == M and w.size == H and sh.shape[1] == H and sc.shape[1] == H
    assert M == 0 or (idx.min() >= 0 and idx.max() < min(sh.shape[0], sc.shape[0]))
    h = np.empty((M, H), dtype=np.uint16)
    q = np.empty((M, H), dtype=np.uint8)
    s = np.empty((M,), dtype=np.float32)
    lib().oracle_rms_quant(_p(x), H, _p(w), _p(sh), ldsh, _p(sc), ldsc, _p(idx), M, H, float(eps), _p(h), _p(q),
                           _p(s))
    return h, q, s


def gate_rms_quant(residual_bits, gate_bits, branch_bits, weight_bits, shift_bits, scale_bits, indices, eps: float):
    """bf16 residual / branch [M, H], gate / shift / scale [B, H] tables, weight [H], indices [M] ->
    (residual_out bf16 bits [M, H], h bf16 bits [M, H], fp8 codes [M, H], fp32 scale [M])."""
    r = _u16(residual_bits)
    M, H = r.shape
    br = _u16(branch_bits)
    w = _u16(weight_bits).reshape(-1)
    g, ldg = _table(gate_bits)
    sh, ldsh = _table(shift_bits)
    sc, ldsc = _table(scale_bits)
    idx = np.ascontiguousarray(np.asarray(indices).reshape(-1), dtype=np.int64)
    assert idx.size == M and w.size == H and br.shape == (M, H) and g.shape[1] == sh.shape[1] == sc.shape[1] == H
    assert M == 0 or (idx.min() >= 0 and idx.max() < min(g.shape[0], sh.shape[0], sc.shape[0]))
    ro = np.empty((M, H), dtype=np.uint16)
    h = np.empty((M, H), dtype=np.uint16)
    q = np.empty((M, H), dtype=np.uint8)
    s = np.empty((M,), dtype=np.float32)
    lib().oracle_gate_rms_quant(_p(r), H, _p(g), ldg, _p(br), H, _p(w), _p(sh), ldsh, _p(sc), ldsc, _p(idx), M, H,
                                float(eps), _p(ro), _p(h), _p(q), _p(s))
    return ro, h, q, s


def qk_norm_rope(x_bits: np.ndarray, weight_bits: np.ndarray, table: np.ndarray, eps: float) -> np.ndarray:
    """bf16 heads [T, heads, 128] (bit patterns), norm weight [128], rope table [T, 96] (its fp32 values: cos | sin)
    -> bf16 bits [T, heads, 128]."""
    x = _u16(x_bits)
    T, heads, D = x.shape
    assert D == 128
    w = _u16(weight_bits).reshape(-1)
    tb = np.ascontiguousarray(table, dtype=np.float32)
    assert w.size == 128 and tb.shape == (T, 96)
    out = np.empty_like(x)
    lib().oracle_qk_norm_rope(_p(x), T, heads, _p(w), _p(tb), float(eps), _p(out))
    return out
