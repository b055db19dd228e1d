"""Torch-facing launchers of the HIP kernels (allocation with torch on the current stream, raw pointers to the C ABI).

Every function here runs the gfx950 kernels of libh3fp8 on the tensors' device and current stream; there is no CPU or
PyTorch fallback.  Shapes, dtypes and strides are checked here and again by the C side.

Layouts follow the reference's vLLM call contract (h3_tp2/fp8_gemm.py:362-373): activations ``a`` e4m3fn [M, K]
row-major; weights as vLLM's ``b`` [K, N] whose transpose ``w = b.t()`` is a row-major [N, K] tensor; per-token scales
[M, 1] / [M] / scalar; per-channel scales [N] / [1, N] / scalar; bf16 or fp16 output.
"""
from __future__ import annotations

import ctypes

import torch

from . import _lib

E4M3 = torch.float8_e4m3fn
FP8_MAX = 448.0
MIN_SCALE = 1.0 / (FP8_MAX * 512.0)     # vLLM's minimum per-token scale (fp8_quant_fuse.py:78-79)

_DT = {torch.bfloat16: _lib.H3FP8_DT_BF16, torch.float16: _lib.H3FP8_DT_FP16, torch.float32: _lib.H3FP8_DT_F32}


_RAW_STREAM = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def _stream(t: torch.Tensor) -> int:
    """The raw HIP stream of torch's current stream on ``t``'s device (the launch stream of every call)."""
    if _RAW_STREAM is not None:
        return _RAW_STREAM(t.get_device())
    return torch.cuda.current_stream(t.device).cuda_stream


def _need_cuda(*ts: torch.Tensor) -> None:
    for t in ts:
        if t is not None and not t.is_cuda:
            raise ValueError("h3_tp2_amd kernels run on the GPU only; got a CPU tensor")


def _rows(t: torch.Tensor, name: str) -> int:
    """Row stride of a 2-D tensor whose rows are contiguous."""
    if t.dim() != 2 or (t.shape[1] > 1 and t.stride(1) != 1):
        raise ValueError(f"{name} must be 2-D with contiguous rows, got shape {tuple(t.shape)} strides {t.stride()}")
    return t.stride(0) if t.shape[0] > 1 else max(t.shape[1], t.stride(0))


def check_buffer(t: torch.Tensor, name: str, shape: tuple, dtype: torch.dtype, device: torch.device,
                 contiguous: bool = False) -> None:
    """A caller-supplied output or workspace must be exactly what the kernel will write: the shape, dtype and device
    given, rows contiguous (or the whole tensor, with ``contiguous``).  A wrong buffer raises here, before any launch,
    instead of becoming an out-of-bounds device write."""
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a tensor, got {type(t).__name__}")
    if t.device != device:
        raise ValueError(f"{name} is on {t.device}, expected {device}")
    if t.dtype != dtype:
        raise ValueError(f"{name} must be {dtype}, got {t.dtype}")
    if tuple(t.shape) != tuple(shape):
        raise ValueError(f"{name} must have shape {tuple(shape)}, got {tuple(t.shape)}")
    if contiguous and not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")
    if t.dim() == 2:
        _rows(t, name)


def _scale_out(t: torch.Tensor, name: str, M: int, device: torch.device) -> None:
    """A per-token scale output: M fp32 entries, contiguous, viewed as [M, 1] or [M]."""
    shape = tuple(t.shape) if isinstance(t, torch.Tensor) else None
    if shape not in ((M, 1), (M,)):
        raise ValueError(f"{name} must have shape ({M}, 1) or ({M},), got {shape}")
    check_buffer(t, name, shape, torch.float32, device, contiguous=True)


def scale_vec(scale: torch.Tensor, n: int, name: str) -> tuple[torch.Tensor, int]:
    """(fp32 tensor, element stride) for a per-row/per-column scale of n entries, or a scalar (stride 0)."""
    if scale.dtype != torch.float32:
        raise ValueError(f"{name} must be float32, got {scale.dtype}")
    s = scale.reshape(-1)
    if s.numel() == 1:
        return s, 0
    if s.numel() != n:
        raise ValueError(f"{name} has {s.numel()} entries, expected {n} or 1")
    return s, s.stride(0)


def init(device=None) -> None:  # noqa: ANN001
    """One-time set-up of the device (the SiLU table); later calls return at once."""
    with torch.cuda.device(device if device is not None else torch.cuda.current_device()):
        _lib.call("h3fp8_init")


# ---- kernel 1 -------------------------------------------------------------------------------------------------------

def quant_rows(x: torch.Tensor, q: torch.Tensor | None = None, scale: torch.Tensor | None = None):
    """Dynamic per-token quant of a bf16 [M, K] tensor: (q e4m3fn [M, K], scale fp32 [M, 1]).
    Replaces ``QuantFP8.forward`` / ``fp8_quant_fuse.quant`` (h3_tp2/fp8_quant_fuse.py:318-327)."""
    _need_cuda(x)
    if x.dtype != torch.bfloat16:
        raise ValueError(f"quant_rows takes bf16, got {x.dtype}")
    M, K = x.shape
    ldx = _rows(x, "x")
    if q is None:
        q, ldq = torch.empty((M, K), device=x.device, dtype=E4M3), K
    else:
        check_buffer(q, "q", (M, K), E4M3, x.device)
        ldq = _rows(q, "q")
    if scale is None:
        scale = torch.empty((M, 1), device=x.device, dtype=torch.float32)
    else:
        _scale_out(scale, "scale", M, x.device)
    _lib.call("h3fp8_quant_rows", x.data_ptr(), ldx, M, K, q.data_ptr(), ldq, scale.data_ptr(), _stream(x))
    return q, scale


def quant_rows_amax(x: torch.Tensor, row_amax: torch.Tensor, q: torch.Tensor | None = None,
                    scale: torch.Tensor | None = None):
    """Per-token quant of bf16 [M, K] with the row maxima given (the tail pass of a fused-amax GEMM)."""
    _need_cuda(x, row_amax)
    if x.dtype != torch.bfloat16 or x.dim() != 2:
        raise ValueError(f"quant_rows_amax takes bf16 [M, K], got {x.dtype} {tuple(x.shape)}")
    M, K = x.shape
    check_buffer(row_amax, "row_amax", (M,), torch.float32, x.device, contiguous=True)
    if q is None:
        q = torch.empty((M, K), device=x.device, dtype=E4M3)
    check_buffer(q, "q", (M, K), E4M3, x.device)
    if scale is None:
        scale = torch.empty((M, 1), device=x.device, dtype=torch.float32)
    _scale_out(scale, "scale", M, x.device)
    _lib.call("h3fp8_quant_rows_amax", x.data_ptr(), _rows(x, "x"), M, K, row_amax.data_ptr(), q.data_ptr(),
              _rows(q, "q"), scale.data_ptr(), _stream(x))
    return q, scale


def quant_segments(base: torch.Tensor, m: int, p: int, seg: int, stride_p: int, stride_m: int):
    """Per-token FP8 quant of M rows whose row m is the P segments ``base[p*stride_p + m*stride_m : +seg]`` (element
    offsets from ``base``'s data pointer, bf16): (q [M, P*seg] e4m3fn contiguous, scale [M, 1] fp32)
    (h3_tp2/ulysses_outq.py:109-124)."""
    _need_cuda(base)
    if base.dtype != torch.bfloat16:
        raise ValueError(f"quant_segments takes bf16, got {base.dtype}")
    if not base.is_contiguous():
        raise ValueError("quant_segments: base must be contiguous (segments are element offsets from its start)")
    if m > 0 and (p - 1) * stride_p + (m - 1) * stride_m + seg > base.numel():
        raise ValueError("quant_segments: the segments reach past the source tensor")
    q = torch.empty((m, p * seg), device=base.device, dtype=E4M3)
    s = torch.empty((m, 1), device=base.device, dtype=torch.float32)
    _lib.call("h3fp8_quant_segments", base.data_ptr(), p, seg, stride_p, stride_m, m, q.data_ptr(), p * seg,
              s.data_ptr(), _stream(base))
    return q, s


def quant_from_recv(recv: torch.Tensor):
    """recv [P, M, hl, d] contiguous (a reverse all-to-all's receive buffer) -> the quant of the [M, P*hl*d] tensor the
    unpack would have produced (row m = recv[0, m], recv[1, m], ...) (h3_tp2/ulysses_outq.py:138-143,
    fp8_quant_fuse.py:372-385)."""
    if recv.dim() != 4 or not recv.is_contiguous():
        raise ValueError("recv must be a contiguous [P, M, hl, d] tensor")
    p, m, hl, d = recv.shape
    seg = hl * d
    return quant_segments(recv, m, p, seg, m * seg, seg)


# ---- kernel 2 -------------------------------------------------------------------------------------------------------

def _gemm_args(a: torch.Tensor, w: torch.Tensor, scale_a: torch.Tensor, scale_b: torch.Tensor, n_cols: int):
    _need_cuda(a, w, scale_a, scale_b)
    if a.dtype != E4M3 or w.dtype != E4M3:
        raise ValueError("a and w must be float8_e4m3fn")
    if a.dim() != 2 or w.dim() != 2 or a.shape[1] != w.shape[1]:
        raise ValueError(f"shape mismatch: a {tuple(a.shape)}, w {tuple(w.shape)} (w is [N, K])")
    M = a.shape[0]
    sa, sa_st = scale_vec(scale_a, M, "scale_a")
    sb, sb_st = scale_vec(scale_b, n_cols, "scale_b")
    return M, sa, sa_st, sb, sb_st


def gemm(a: torch.Tensor, w: torch.Tensor, scale_a: torch.Tensor, scale_b: torch.Tensor,
         out_dtype: torch.dtype = torch.bfloat16, bias: torch.Tensor | None = None, out: torch.Tensor | None = None,
         row_amax: torch.Tensor | None = None) -> torch.Tensor:
    """y [M, N] = round(sa[m] * (sb[n] * (a @ w.T)[m, n])) (+ bias by one fma); ``w`` is the [N, K] weight.
    With ``row_amax`` ([M] fp32) the epilogue also reduces max |y| per row (for the next layer's quant).
    ``out_dtype=torch.float32`` returns the raw fp32 accumulator (scales ignored: the two-pass form's product, whose
    scale pass or fused consumer follows; the reference's OUT 0)."""
    N = w.shape[0]
    M, sa, sa_st, sb, sb_st = _gemm_args(a, w, scale_a, scale_b, N)
    if out_dtype not in _DT:
        raise ValueError(f"out_dtype must be bf16, fp16 or fp32 (the raw accumulator), got {out_dtype}")
    if bias is not None and (bias.dim() != 1 or bias.numel() != N or bias.dtype != out_dtype
                             or bias.device != a.device or not bias.is_contiguous()):
        raise ValueError("bias must be a contiguous [N] vector in the output dtype on the operands' device")
    if out is None:
        y, ldy = torch.empty((M, N), device=a.device, dtype=out_dtype), N
    else:
        y = out
        check_buffer(y, "out", (M, N), out_dtype, a.device)
        ldy = _rows(y, "y")
    if row_amax is not None:
        check_buffer(row_amax, "row_amax", (M,), torch.float32, a.device, contiguous=True)
    _lib.call("h3fp8_gemm", a.data_ptr(), _rows(a, "a"), w.data_ptr(), _rows(w, "w"), sa.data_ptr(), sa_st,
              sb.data_ptr(), sb_st, bias.data_ptr() if bias is not None else None, y.data_ptr(), ldy,
              _DT[out_dtype], M, N, a.shape[1], row_amax.data_ptr() if row_amax is not None else None, _stream(a))
    return y


def _scale_ptr(scale: torch.Tensor) -> tuple[int, int]:
    """(pointer, element stride) of a scale of 1 or n entries already sized by the caller's eligibility test: a scalar
    has stride 0; [n], [n, 1] and [1, n] views are read in place; any other layout through a flattened view."""
    if scale.numel() == 1:
        return scale.data_ptr(), 0
    if scale.dim() == 1 or (scale.dim() == 2 and scale.shape[1] == 1):
        return scale.data_ptr(), scale.stride(0)
    if scale.dim() == 2 and scale.shape[0] == 1:
        return scale.data_ptr(), scale.stride(1)
    flat = scale.reshape(-1)
    return flat.data_ptr(), flat.stride(0)


def scaled_mm_eligible(a: torch.Tensor, b: torch.Tensor, scale_a: torch.Tensor, scale_b: torch.Tensor,
                       out_dtype: torch.dtype, bias: torch.Tensor | None = None) -> torch.Tensor:
    """Kernel 2 on a call that passed ``fp8_gemm.eligible`` -- the dispatcher's lean host path.  That test has checked
    the dtypes (e4m3 operands, fp32 scales, bf16 / fp16 out), the shapes, ``a`` contiguous, ``b.t()`` contiguous, the
    scale and bias sizes and K, N multiples of 16; what it leaves -- every operand on ``a``'s GPU, a bias in the
    output dtype -- is checked here, and the C side checks sizes, strides and alignment again before any launch."""
    dev = a.device
    if not a.is_cuda:
        raise ValueError("h3_tp2_amd kernels run on the GPU only; got a CPU tensor")
    if scale_a.device != dev or scale_b.device != dev or (bias is not None and bias.device != dev):
        raise ValueError("scaled_mm: every operand must be on the same GPU")
    M, K = a.shape
    N = b.shape[1]
    if bias is not None and (bias.dtype != out_dtype or not bias.is_contiguous()):
        bias = bias.to(out_dtype).contiguous()
    sa, sa_st = _scale_ptr(scale_a)
    sb, sb_st = _scale_ptr(scale_b)
    y = torch.empty((M, N), device=dev, dtype=out_dtype)
    _lib.call("h3fp8_gemm", a.data_ptr(), K, b.data_ptr(), K, sa, sa_st, sb, sb_st,
              bias.data_ptr() if bias is not None else None, y.data_ptr(), N, _DT[out_dtype], M, N, K, None,
              _stream(a))
    return y


def scaled_mm(a: torch.Tensor, b: torch.Tensor, scale_a: torch.Tensor, scale_b: torch.Tensor, out_dtype: torch.dtype,
              bias: torch.Tensor | None = None) -> torch.Tensor:
    """``ops.cutlass_scaled_mm(a, b, scale_a, scale_b, out_dtype, bias)`` with vLLM's ``b`` [K, N] (``b.t()``
    contiguous): the HIP GEMM (h3_tp2/fp8_gemm.py:149-164 / fp8_cutlass.py:115-131 contract)."""
    return gemm(a, b.t(), scale_a, scale_b, out_dtype, bias)


def gemm_quant(a: torch.Tensor, w: torch.Tensor, scale_a: torch.Tensor, scale_b: torch.Tensor,
               bias: torch.Tensor | None = None):
    """GEMM to bf16 y plus the per-token e4m3 quant of y fused through the epilogue's row maxima:
    returns (y bf16 [M, N], q e4m3fn [M, N], scale fp32 [M, 1])."""
    N = w.shape[0]
    M, sa, sa_st, sb, sb_st = _gemm_args(a, w, scale_a, scale_b, N)
    _check_bias(bias, N, a.device)
    dev = a.device
    y = torch.empty((M, N), device=dev, dtype=torch.bfloat16)
    amax = torch.empty((M,), device=dev, dtype=torch.float32)
    q = torch.empty((M, N), device=dev, dtype=E4M3)
    s = torch.empty((M, 1), device=dev, dtype=torch.float32)
    _lib.call("h3fp8_gemm_quant", a.data_ptr(), _rows(a, "a"), w.data_ptr(), _rows(w, "w"), sa.data_ptr(), sa_st,
              sb.data_ptr(), sb_st, bias.data_ptr() if bias is not None else None, y.data_ptr(), N, M, N, a.shape[1],
              amax.data_ptr(), q.data_ptr(), N, s.data_ptr(), _stream(a))
    return y, q, s


# ---- kernel 3 -------------------------------------------------------------------------------------------------------

def _check_bias(bias: torch.Tensor | None, n: int, device: torch.device) -> None:
    """A bf16 bias of n entries (kernel 3 reads 2F: gate then up), contiguous, on the operands' device."""
    if bias is None:
        return
    if not isinstance(bias, torch.Tensor) or bias.dim() != 1 or bias.numel() != n or bias.dtype != torch.bfloat16 \
            or bias.device != device or not bias.is_contiguous():
        raise ValueError(f"bias must be a contiguous bfloat16 [{n}] vector on {device}")


def _gate_up_width(w_gate_up: torch.Tensor) -> int:
    F2 = w_gate_up.shape[0]
    if F2 % 2:
        raise ValueError("gate/up weight must have an even number of rows")
    return F2 // 2

def gemm_swiglu(a: torch.Tensor, w_gate_up: torch.Tensor, scale_a: torch.Tensor, scale_b: torch.Tensor,
                bias: torch.Tensor | None = None, row_amax: torch.Tensor | None = None,
                out: torch.Tensor | None = None) -> torch.Tensor:
    """fc1 + epilogue + SwiGLU in one kernel: bf16 h [M, F] from a [M, K] and the merged [2F, K] gate|up weight
    (h3_tp2/fp8_swiglu.py:230-241).  ``out``: a caller-supplied h (bf16 [M, F], rows contiguous)."""
    F = _gate_up_width(w_gate_up)
    M, sa, sa_st, sb, sb_st = _gemm_args(a, w_gate_up, scale_a, scale_b, 2 * F)
    _check_bias(bias, 2 * F, a.device)
    if row_amax is not None:
        check_buffer(row_amax, "row_amax", (M,), torch.float32, a.device, contiguous=True)
    h = out if out is not None else torch.empty((M, F), device=a.device, dtype=torch.bfloat16)
    check_buffer(h, "out", (M, F), torch.bfloat16, a.device)
    _lib.call("h3fp8_gemm_swiglu", a.data_ptr(), _rows(a, "a"), w_gate_up.data_ptr(), _rows(w_gate_up, "w"),
              sa.data_ptr(), sa_st, sb.data_ptr(), sb_st, bias.data_ptr() if bias is not None else None, h.data_ptr(),
              _rows(h, "out"), row_amax.data_ptr() if row_amax is not None else None, M, F, a.shape[1], _stream(a))
    return h


def gemm_swiglu_quant(a: torch.Tensor, w_gate_up: torch.Tensor, scale_a: torch.Tensor, scale_b: torch.Tensor,
                      bias: torch.Tensor | None = None, h_ws: torch.Tensor | None = None):
    """fc1 + SwiGLU + per-token requant (fp8_swiglu level 2, h3_tp2/fp8_swiglu.py:191-200): (q [M, F], scale [M, 1])."""
    F = _gate_up_width(w_gate_up)
    M, sa, sa_st, sb, sb_st = _gemm_args(a, w_gate_up, scale_a, scale_b, 2 * F)
    _check_bias(bias, 2 * F, a.device)
    dev = a.device
    if h_ws is None:
        h_ws = torch.empty((M, F), device=dev, dtype=torch.bfloat16)
    check_buffer(h_ws, "h_ws", (M, F), torch.bfloat16, dev, contiguous=True)   # the C side writes rows of F
    amax = torch.empty((M,), device=dev, dtype=torch.float32)
    q = torch.empty((M, F), device=dev, dtype=E4M3)
    s = torch.empty((M, 1), device=dev, dtype=torch.float32)
    _lib.call("h3fp8_gemm_swiglu_quant", a.data_ptr(), _rows(a, "a"), w_gate_up.data_ptr(), _rows(w_gate_up, "w"),
              sa.data_ptr(), sa_st, sb.data_ptr(), sb_st, bias.data_ptr() if bias is not None else None, M, F,
              a.shape[1], h_ws.data_ptr(), amax.data_ptr(), q.data_ptr(), F, s.data_ptr(), _stream(a))
    return q, s


def _product_in(x32: torch.Tensor, name: str = "x32") -> tuple[int, int]:
    """An fp32 product [M, W] with contiguous rows: (M, W).  The scale passes read it as fp32, so any other dtype
    would make them read past its allocation; it is refused here, before any launch."""
    if not isinstance(x32, torch.Tensor) or x32.dim() != 2:
        raise ValueError(f"{name} must be a 2-D tensor")
    if x32.dtype != torch.float32:
        raise ValueError(f"{name} must be float32 (the raw GEMM product), got {x32.dtype}")
    _rows(x32, name)
    return x32.shape[0], x32.shape[1]


def _swiglu_width(W: int, name: str) -> int:
    """F of a [gate | up] row of width W = 2F; the kernels take F in multiples of 4."""
    if W % 2 or (W // 2) % 4:
        raise ValueError(f"{name} must have an even width 2F with F a multiple of 4, got width {W}")
    return W // 2


def _epi_scales(x32: torch.Tensor, sa: torch.Tensor, sb: torch.Tensor, width: int):
    M = x32.shape[0]
    s_a, sa_st = scale_vec(sa, M, "sa")
    s_b, sb_st = scale_vec(sb, width, "sb")
    return s_a, sa_st, s_b, sb_st


def scale_swiglu(x32: torch.Tensor, sa: torch.Tensor, sb: torch.Tensor, bias: torch.Tensor | None = None):
    """fp32 product [M, 2F] -> bf16 SwiGLU [M, F] (h3_tp2/fp8_swiglu.py:180-188)."""
    _need_cuda(x32, sa, sb)
    M, W = _product_in(x32)
    F = _swiglu_width(W, "x32")
    s_a, sa_st, s_b, sb_st = _epi_scales(x32, sa, sb, W)
    _check_bias(bias, W, x32.device)
    h = torch.empty((M, F), device=x32.device, dtype=torch.bfloat16)
    _lib.call("h3fp8_scale_swiglu", x32.data_ptr(), _rows(x32, "x32"), s_a.data_ptr(), sa_st, s_b.data_ptr(), sb_st,
              bias.data_ptr() if bias is not None else None, M, F, h.data_ptr(), F, _stream(x32))
    return h


def scale_swiglu_quant(x32: torch.Tensor, sa: torch.Tensor, sb: torch.Tensor, bias: torch.Tensor | None = None):
    """fp32 product [M, 2F] -> SwiGLU -> per-token quant: (q [M, F], scale [M, 1]) (h3_tp2/fp8_swiglu.py:191-200)."""
    _need_cuda(x32, sa, sb)
    M, W = _product_in(x32)
    F = _swiglu_width(W, "x32")
    s_a, sa_st, s_b, sb_st = _epi_scales(x32, sa, sb, W)
    _check_bias(bias, W, x32.device)
    q = torch.empty((M, F), device=x32.device, dtype=E4M3)
    s = torch.empty((M, 1), device=x32.device, dtype=torch.float32)
    _lib.call("h3fp8_scale_swiglu_quant", x32.data_ptr(), _rows(x32, "x32"), s_a.data_ptr(), sa_st, s_b.data_ptr(),
              sb_st, bias.data_ptr() if bias is not None else None, M, F, q.data_ptr(), F, s.data_ptr(),
              _stream(x32))
    return q, s


def silu_mul_quant(x: torch.Tensor):
    """silu_and_mul on bf16 [M, 2F] + per-token quant: (q [M, F], scale [M, 1]) (h3_tp2/fp8_quant_fuse.py:392-402)."""
    _need_cuda(x)
    if not isinstance(x, torch.Tensor) or x.dim() != 2 or x.dtype != torch.bfloat16:
        raise ValueError("silu_mul_quant takes a bf16 [M, 2F] tensor")
    M, W = x.shape
    F = _swiglu_width(W, "x")
    if x.shape[0] > 1 and _rows(x, "x") % 8:
        raise ValueError("silu_mul_quant: the row stride of x must be a multiple of 8 elements")
    q = torch.empty((M, F), device=x.device, dtype=E4M3)
    s = torch.empty((M, 1), device=x.device, dtype=torch.float32)
    _lib.call("h3fp8_silu_mul_quant", x.data_ptr(), _rows(x, "x"), M, F, q.data_ptr(), F, s.data_ptr(), _stream(x))
    return q, s


# ---- the quant fused into its producers --------------------------------------------------------------------------

def _producer_args(x: torch.Tensor, weight: torch.Tensor, tables: tuple, indices: torch.Tensor, names: tuple):
    """Checks shared by the two producers: bf16 rows, weight [H], [B, H] tables, indices int32/int64 [M]."""
    _need_cuda(x, weight, indices, *tables)
    M, H = x.shape
    for t, n in ((x, "x"), *zip(tables, names)):
        if t.dtype != torch.bfloat16:
            raise ValueError(f"{n} must be bfloat16, got {t.dtype}")
        _rows(t, n)
    if weight.dtype != torch.bfloat16 or weight.numel() != H or (H > 1 and weight.reshape(-1).stride(0) != 1):
        raise ValueError(f"weight must be a contiguous bfloat16 [{H}] vector")
    n_index = min(t.shape[0] for t in tables)
    if any(t.shape[1] != H for t in tables):
        raise ValueError(f"{', '.join(names)} must have {H} columns")
    if indices.dim() != 1 or indices.shape[0] != M or indices.dtype not in (torch.int32, torch.int64):
        raise ValueError(f"indices must be int32/int64 [{M}], got {indices.dtype} {tuple(indices.shape)}")
    return M, H, n_index, indices.element_size()


def _placeholder(ph: torch.Tensor | None, like: torch.Tensor) -> tuple[int | None, int]:
    if ph is None:
        return None, 0
    if ph.shape != like.shape or ph.dtype != torch.bfloat16 or ph.device != like.device:
        raise ValueError(f"ph must be bfloat16 {tuple(like.shape)} on {like.device}")
    return ph.data_ptr(), _rows(ph, "ph")


def rms_quant(x: torch.Tensor, weight: torch.Tensor, shift: torch.Tensor, scale: torch.Tensor,
              indices: torch.Tensor, eps: float, ph: torch.Tensor | None = None):
    """``rms_norm_indexed_scale_shift`` + the per-token quant of its output: (fp8 [M, H], scale [M, 1]); with ``ph``
    (bf16 [M, H]) the modulated bf16 row is stored there too (h3_tp2/fp8_quant_fuse.py:330-346)."""
    M, H, n_index, ib = _producer_args(x, weight, (shift, scale), indices, ("shift", "scale"))
    q = torch.empty((M, H), device=x.device, dtype=E4M3)
    s = torch.empty((M, 1), device=x.device, dtype=torch.float32)
    _lib.call("h3fp8_rms_quant", x.data_ptr(), _rows(x, "x"), weight.data_ptr(), shift.data_ptr(),
              _rows(shift, "shift"), scale.data_ptr(), _rows(scale, "scale"), n_index, indices.data_ptr(),
              indices.stride(0), ib, M, H, float(eps), q.data_ptr(), H, s.data_ptr(), *_placeholder(ph, x), _stream(x))
    return q, s


def rms_norm_indexed_scale_shift(x: torch.Tensor, weight: torch.Tensor, shift: torch.Tensor, scale: torch.Tensor,
                                 indices: torch.Tensor, eps: float) -> torch.Tensor:
    """The producer alone (bf16 h [M, H], no quant), with the fused form's arithmetic: the drop-in for the stock
    ``rms_norm_indexed_scale_shift`` (tests/fake_h3_consumers.py:77-84 states its formula)."""
    M, H, n_index, ib = _producer_args(x, weight, (shift, scale), indices, ("shift", "scale"))
    h = torch.empty((M, H), device=x.device, dtype=torch.bfloat16)
    _lib.call("h3fp8_rms_quant", x.data_ptr(), _rows(x, "x"), weight.data_ptr(), shift.data_ptr(),
              _rows(shift, "shift"), scale.data_ptr(), _rows(scale, "scale"), n_index, indices.data_ptr(),
              indices.stride(0), ib, M, H, float(eps), None, 0, None, h.data_ptr(), H, _stream(x))
    return h


def indexed_gate_rms_norm_scale_shift(residual: torch.Tensor, gate: torch.Tensor, branch: torch.Tensor,
                                      weight: torch.Tensor, shift: torch.Tensor, scale: torch.Tensor,
                                      indices: torch.Tensor, eps: float) -> tuple[torch.Tensor, torch.Tensor]:
    """The gated producer alone: (residual_out bf16 [M, H], h bf16 [M, H]) with the fused form's arithmetic
    (tests/fake_h3_consumers.py:66-74 states its formula)."""
    M, H, n_index, ib = _producer_args(residual, weight, (gate, shift, scale), indices, ("gate", "shift", "scale"))
    if branch.shape != residual.shape or branch.dtype != torch.bfloat16:
        raise ValueError("branch must be bfloat16 with the residual's shape")
    _need_cuda(branch)
    res = torch.empty((M, H), device=residual.device, dtype=torch.bfloat16)
    h = torch.empty((M, H), device=residual.device, dtype=torch.bfloat16)
    _lib.call("h3fp8_gate_rms_quant", residual.data_ptr(), _rows(residual, "residual"), gate.data_ptr(),
              _rows(gate, "gate"), branch.data_ptr(), _rows(branch, "branch"), weight.data_ptr(), shift.data_ptr(),
              _rows(shift, "shift"), scale.data_ptr(), _rows(scale, "scale"), n_index, indices.data_ptr(),
              indices.stride(0), ib, M, H, float(eps), res.data_ptr(), H, None, 0, None, h.data_ptr(), H,
              _stream(residual))
    return res, h


def gate_rms_quant(residual: torch.Tensor, gate: torch.Tensor, branch: torch.Tensor, weight: torch.Tensor,
                   shift: torch.Tensor, scale: torch.Tensor, indices: torch.Tensor, eps: float,
                   ph: torch.Tensor | None = None):
    """``indexed_gate_rms_norm_scale_shift`` with the modulated output quantised per token: (residual_out bf16 [M, H],
    fp8 [M, H], scale [M, 1]); ``ph`` as in ``rms_quant`` (h3_tp2/fp8_quant_fuse.py:349-369)."""
    M, H, n_index, ib = _producer_args(residual, weight, (gate, shift, scale), indices, ("gate", "shift", "scale"))
    if branch.shape != residual.shape or branch.dtype != torch.bfloat16:
        raise ValueError("branch must be bfloat16 with the residual's shape")
    _need_cuda(branch)
    res = torch.empty((M, H), device=residual.device, dtype=torch.bfloat16)
    q = torch.empty((M, H), device=residual.device, dtype=E4M3)
    s = torch.empty((M, 1), device=residual.device, dtype=torch.float32)
    _lib.call("h3fp8_gate_rms_quant", residual.data_ptr(), _rows(residual, "residual"), gate.data_ptr(),
              _rows(gate, "gate"), branch.data_ptr(), _rows(branch, "branch"), weight.data_ptr(), shift.data_ptr(),
              _rows(shift, "shift"), scale.data_ptr(), _rows(scale, "scale"), n_index, indices.data_ptr(),
              indices.stride(0), ib, M, H, float(eps), res.data_ptr(), H, q.data_ptr(), H, s.data_ptr(),
              *_placeholder(ph, residual), _stream(residual))
    return res, q, s


# ---- consumers of a two-pass GEMM's fp32 product (the scale pass fused in) ----------------------------------------

def _product_args(x32: torch.Tensor, sa: torch.Tensor, sb: torch.Tensor, bias: torch.Tensor | None, M: int, N: int):
    """The fp32 product [M, >= N] and contiguous sa [M] / sb [N] fp32 vectors (scalars broadcast), bias bf16 [N]."""
    _need_cuda(x32, sa, sb, bias)
    if x32.dtype != torch.float32 or x32.dim() != 2 or x32.shape[0] != M or x32.shape[1] < N:
        raise ValueError(f"the product must be fp32 [{M}, >= {N}], got {x32.dtype} {tuple(x32.shape)}")
    s_a = sa.reshape(-1).float()
    s_a = (s_a.expand(M) if s_a.numel() == 1 else s_a).contiguous()
    s_b = sb.reshape(-1).float()
    s_b = (s_b.expand(x32.shape[1]) if s_b.numel() == 1 else s_b).contiguous()
    if s_a.numel() != M or s_b.numel() < N:
        raise ValueError("scale vectors do not match the product")
    if bias is not None and (bias.dtype != torch.bfloat16 or bias.dim() != 1 or bias.numel() < N
                             or not bias.is_contiguous()):
        raise ValueError("bias must be a contiguous bf16 vector")
    return s_a, s_b


def scale_gate_rms_quant(x32: torch.Tensor, sa: torch.Tensor, sb: torch.Tensor, bias: torch.Tensor | None,
                         residual: torch.Tensor, gate: torch.Tensor, weight: torch.Tensor, shift: torch.Tensor,
                         scale: torch.Tensor, indices: torch.Tensor, eps: float, residual_out: torch.Tensor | None = None,
                         quant: bool = False, modulated: bool = True):
    """``indexed_gate_rms_norm_scale_shift(residual, gate, branch, ...)`` with branch = the scale pass of the fp32
    product ``x32`` (h3_tp2/fp8_consumers.py:464-485): (residual_out, modulated bf16) and, with ``quant``, the per-token
    e4m3 quant of the modulated row as well: (residual_out, q, scale[, modulated])."""
    M, H, n_index, ib = _producer_args(residual, weight, (gate, shift, scale), indices, ("gate", "shift", "scale"))
    s_a, s_b = _product_args(x32, sa, sb, bias, M, H)
    res = residual_out if residual_out is not None else torch.empty((M, H), device=residual.device,
                                                                    dtype=torch.bfloat16)
    check_buffer(res, "residual_out", (M, H), torch.bfloat16, residual.device)
    h = torch.empty((M, H), device=residual.device, dtype=torch.bfloat16) if modulated or not quant else None
    q = torch.empty((M, H), device=residual.device, dtype=E4M3) if quant else None
    s = torch.empty((M, 1), device=residual.device, dtype=torch.float32) if quant else None
    _lib.call("h3fp8_scale_gate_rms_quant", x32.data_ptr(), _rows(x32, "x32"), s_a.data_ptr(), s_b.data_ptr(),
              bias.data_ptr() if bias is not None else None, residual.data_ptr(), _rows(residual, "residual"),
              gate.data_ptr(), _rows(gate, "gate"), weight.data_ptr(), shift.data_ptr(), _rows(shift, "shift"),
              scale.data_ptr(), _rows(scale, "scale"), n_index, indices.data_ptr(), indices.stride(0), ib, M, H,
              float(eps), res.data_ptr(), _rows(res, "residual_out"), q.data_ptr() if q is not None else None,
              H, s.data_ptr() if s is not None else None, h.data_ptr() if h is not None else None, H,
              _stream(residual))
    if quant:
        return (res, q, s, h) if h is not None else (res, q, s)
    return res, h


def scale_indexed_gate(x32: torch.Tensor, sa: torch.Tensor, sb: torch.Tensor, bias: torch.Tensor | None,
                       x: torch.Tensor, gate: torch.Tensor, indices: torch.Tensor,
                       out: torch.Tensor | None = None) -> torch.Tensor:
    """``indexed_gate(x, gate, other, indices)`` = bf16(x + gate[indices] * other) with other = the scale pass of the
    fp32 product ``x32`` (h3_tp2/fp8_consumers.py:488-504)."""
    _need_cuda(x, gate, indices)
    M, H = x.shape
    if x.dtype != torch.bfloat16 or gate.dtype != torch.bfloat16 or gate.dim() != 2 or gate.shape[1] != H:
        raise ValueError("x and gate must be bf16 with the same width")
    if indices.dim() != 1 or indices.shape[0] != M or indices.dtype not in (torch.int32, torch.int64):
        raise ValueError(f"indices must be int32/int64 [{M}]")
    s_a, s_b = _product_args(x32, sa, sb, bias, M, H)
    o = out if out is not None else torch.empty((M, H), device=x.device, dtype=torch.bfloat16)
    check_buffer(o, "out", (M, H), torch.bfloat16, x.device)
    _lib.call("h3fp8_scale_indexed_gate", x32.data_ptr(), _rows(x32, "x32"), s_a.data_ptr(), s_b.data_ptr(),
              bias.data_ptr() if bias is not None else None, x.data_ptr(), _rows(x, "x"), gate.data_ptr(),
              _rows(gate, "gate"), gate.shape[0], indices.data_ptr(), indices.stride(0), indices.element_size(), M, H,
              o.data_ptr(), _rows(o, "out"), _stream(x))
    return o


def scale_qk_norm_rope(x32: torch.Tensor, sa: torch.Tensor, sb: torch.Tensor, bias: torch.Tensor | None,
                       num_heads: int, num_kv_heads: int, q_weight: torch.Tensor, k_weight: torch.Tensor,
                       rope_table: torch.Tensor, eps: float, v_out: torch.Tensor | None = None):
    """q, k of ``fused_qk_norm_rope`` (head_dim 128, rotary 96, half-split) on the qkv GEMM's fp32 product: the q heads
    are product columns [0, 128 H), the k heads the next 128 Hk.  Returns (q [T, H, 128], k [T, Hk, 128]) bf16
    (h3_tp2/fp8_consumers.py:424-461).  With ``v_out`` (bf16 [T, Hv, 128], dims contiguous) the Hv heads after the k
    heads get the scale pass into it in the same launch, the bytes ``scale_bias_cast`` writes
    (h3_tp2/fp8_consumers.py:373-380)."""
    T = x32.shape[0]
    Hv = 0
    if v_out is not None:
        if v_out.dtype != torch.bfloat16 or v_out.dim() != 3 or v_out.shape[0] != T or v_out.shape[2] != 128 \
                or v_out.stride(2) != 1 or v_out.device != x32.device:
            raise ValueError(f"v_out must be bf16 [{T}, Hv, 128] on the product's device with contiguous dims")
        Hv = v_out.shape[1]
    s_a, s_b = _product_args(x32, sa, sb, bias, T, (num_heads + num_kv_heads + Hv) * 128)
    _need_cuda(q_weight, k_weight, rope_table)
    if rope_table.dim() != 2 or rope_table.shape != (T, 96) or rope_table.stride(1) != 1 \
            or rope_table.dtype not in (torch.float32, torch.bfloat16):
        raise ValueError(f"rope_table must be fp32/bf16 [{T}, 96] with contiguous rows")
    for w in (q_weight, k_weight):
        if w.dtype != torch.bfloat16 or w.numel() != 128 or not w.is_contiguous():
            raise ValueError("q/k norm weights must be contiguous bf16 [128]")
    oq = torch.empty((T, num_heads, 128), device=x32.device, dtype=torch.bfloat16)
    ok = torch.empty((T, num_kv_heads, 128), device=x32.device, dtype=torch.bfloat16)
    _lib.call("h3fp8_scale_qkv_norm_rope", x32.data_ptr(), _rows(x32, "x32"), s_a.data_ptr(), s_b.data_ptr(),
              bias.data_ptr() if bias is not None else None, T, num_heads, num_kv_heads, Hv, q_weight.data_ptr(),
              k_weight.data_ptr(), rope_table.data_ptr(), rope_table.stride(0) if T > 1 else 96,
              int(rope_table.dtype == torch.float32), float(eps), oq.data_ptr(), oq.stride(0), oq.stride(1),
              ok.data_ptr(), ok.stride(0), ok.stride(1), v_out.data_ptr() if Hv else None,
              v_out.stride(0) if Hv else 0, v_out.stride(1) if Hv else 0, _stream(x32))
    return oq, ok


def scale_bias_cast(x32: torch.Tensor, sa: torch.Tensor, sb: torch.Tensor, bias: torch.Tensor | None,
                    out_dtype: torch.dtype, out: torch.Tensor | None = None) -> torch.Tensor:
    """The two-pass scale pass: round(sa * (sb * x32)) (+ bias by one fma) (h3_tp2/fp8_gemm.py:37-54, :167-171)."""
    _need_cuda(x32, sa, sb)
    M, N = _product_in(x32)
    s_a, sa_st, s_b, sb_st = _epi_scales(x32, sa, sb, N)
    if out_dtype not in (torch.bfloat16, torch.float16):
        raise ValueError(f"scale_bias_cast writes bf16 or fp16, got {out_dtype}")
    if bias is not None and (bias.dim() != 1 or bias.numel() != N or bias.dtype != out_dtype
                             or bias.device != x32.device or not bias.is_contiguous()):
        raise ValueError("bias must be a contiguous [N] vector in the output dtype")
    y = out if out is not None else torch.empty((M, N), device=x32.device, dtype=out_dtype)
    check_buffer(y, "out", (M, N), out_dtype, x32.device)
    _lib.call("h3fp8_scale_bias_cast", x32.data_ptr(), _rows(x32, "x32"), s_a.data_ptr(), sa_st, s_b.data_ptr(),
              sb_st, bias.data_ptr() if bias is not None else None, y.data_ptr(), _rows(y, "y"), _DT[out_dtype], M, N,
              _stream(x32))
    return y


# ---- grouped GEMM ---------------------------------------------------------------------------------------------------

def grouped_gemm(problems):  # noqa: ANN001,ANN201
    """Several (a, w, scale_a, scale_b) problems in one launch; returns their bf16 outputs."""
    if len(problems) > _lib.MAX_GROUPS:
        raise ValueError(f"at most {_lib.MAX_GROUPS} groups per launch")
    arr = (_lib.Group * max(1, len(problems)))()
    outs, keep = [], []
    for i, (a, w, scale_a, scale_b) in enumerate(problems):
        N = w.shape[0]
        M, sa, sa_st, sb, sb_st = _gemm_args(a, w, scale_a, scale_b, N)
        y = torch.empty((M, N), device=a.device, dtype=torch.bfloat16)
        outs.append(y)
        keep += [sa, sb]
        arr[i] = _lib.Group(a.data_ptr(), _rows(a, "a"), w.data_ptr(), _rows(w, "w"), sa.data_ptr(), sa_st,
                            sb.data_ptr(), sb_st, y.data_ptr(), N, M, N, a.shape[1])
    if problems:
        _lib.call("h3fp8_grouped_gemm", arr, len(problems), _stream(problems[0][0]))
    return outs


# ---- self-checks ----------------------------------------------------------------------------------------------------

def selfcheck_e4m3() -> tuple[int, int]:
    """(non-NaN mismatches, NaN inputs not mapped to NaN) of the hardware e4m3 cvt against torch's cast rule, over
    every fp32 bit pattern in [-448, 448] and every NaN (synchronous)."""
    bad, nan_bad = ctypes.c_uint64(0), ctypes.c_uint64(0)
    _lib.call("h3fp8_selfcheck_e4m3", ctypes.byref(bad), ctypes.byref(nan_bad))
    return int(bad.value), int(nan_bad.value)


def selfcheck_bf16() -> tuple[int, int]:
    """(non-NaN mismatches, NaN inputs not mapped to NaN) of the hardware bf16 pair conversion against the RNE rule,
    over every fp32 bit pattern (synchronous)."""
    bad, nan_bad = ctypes.c_uint64(0), ctypes.c_uint64(0)
    _lib.call("h3fp8_selfcheck_bf16", ctypes.byref(bad), ctypes.byref(nan_bad))
    return int(bad.value), int(nan_bad.value)


def silu_table(device=None) -> torch.Tensor:  # noqa: ANN001
    """The device's SiLU table (65536 bf16 bit patterns as int16)."""
    dev = torch.device("cuda", torch.cuda.current_device()) if device is None else torch.device(device)
    out = torch.empty(65536, device=dev, dtype=torch.int16)
    with torch.cuda.device(dev):
        _lib.call("h3fp8_copy_silu_table", out.data_ptr(), torch.cuda.current_stream(dev).cuda_stream)
    return out


MFMA_LOOP_FLOP_PER_ROUND = 2.0 * 32 * 32 * 64 * 16 * 4    # per workgroup and round of h3fp8_mfma_loop


def mfma_loop(out: torch.Tensor, iters: int, seed: int = 1) -> float:
    """Launches the register-only FP8 MFMA loop (one workgroup per 256 floats of ``out``, ``iters`` rounds) on the
    current stream and returns its FLOP count: the chip's sustained MFMA rate with no memory traffic."""
    _need_cuda(out)
    if out.dtype != torch.float32 or not out.is_contiguous() or out.numel() % 256 or out.numel() == 0:
        raise ValueError("out must be a contiguous fp32 tensor of a positive multiple of 256 elements")
    blocks = out.numel() // 256
    _lib.call("h3fp8_mfma_loop", out.data_ptr(), blocks, int(iters), int(seed) & 0xffffffff, _stream(out))
    return MFMA_LOOP_FLOP_PER_ROUND * blocks * iters
