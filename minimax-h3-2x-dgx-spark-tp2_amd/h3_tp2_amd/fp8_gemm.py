"""Dispatcher of the row/column-scaled FP8 GEMMs: the drop-in for ``ops.cutlass_scaled_mm`` on MI355X (gfx950).

Mirrors the hook surface of the reference's h3_tp2/fp8_gemm.py -- ``install`` (:344-410) with the eligibility test of
its ``_mm`` (:362-373), ``route`` (:328-341), ``set_router`` / ``set_stash_hook`` (:313-325), ``scaled_mm_tensor32``
(:149-164), ``scaled_mm_fused`` (:240-248), ``unit_scale`` (:132-146), ``_vec_scales`` (:230-237), ``_launch``
(:167-171) and ``_state`` (:117) -- so that the modules which call into it (fp8_consumers, fp8_swiglu,
fp8_quant_fuse, the router of fp8_hip) keep their call sites.  The compute is the HIP kernels of libh3fp8:

* level ``"hip"`` (default): an eligible call runs the routers, then the stash hooks, then kernel 2 -- one launch,
  the per-token x per-channel scale epilogue applied to the fp32 accumulator in registers, no fp32 [M, N] product;
* level ``"tensor32"``: the two-pass contract on the device -- kernel 2 in raw-accumulator mode to an fp32 product,
  then the scale pass ``h3fp8_scale_bias_cast`` -- kept for stash consumers that read the fp32 product;
* every call that fails the eligibility test keeps the stock op it replaced.

There is no CPU or PyTorch fallback for an eligible call: the HIP kernel runs or the call raises.
"""
from __future__ import annotations

import logging
import threading

import torch

from . import _lib, ops

logger = logging.getLogger("h3_tp2_amd.fp8_gemm")

E4M3 = torch.float8_e4m3fn
LEVELS = ("hip", "tensor32", "off")

# level: the level running; fused: an eligible call is one kernel-2 launch (the consumers' stash hooks stand down when
# it is set, as they do for the reference's fused level); triton: the device scale pass is usable (the key name is the
# one fp8_consumers and fp8_swiglu test before calling ``_launch``); selfcheck: failing install-check cases.
_state = {"level": "off", "fused": False, "triton": False, "installed": False, "selfcheck": None}
_stats = {"hip": 0, "two_pass": 0, "stock": 0, "routed": 0, "stashed": 0}
_routers: list = []
_stash_hooks: list = []
_lock = threading.Lock()
_UNIT: dict = {}


def eligible(a, b, scale_a, scale_b, out_dtype, bias=None) -> bool:  # noqa: ANN001
    """The dispatcher's eligibility test (h3_tp2/fp8_gemm.py:364-371): True -> this module computes the call."""
    if a.dim() != 2 or b.dim() != 2 or a.shape[1] != b.shape[0]:
        return False
    M, N = a.shape[0], b.shape[1]
    if scale_a.numel() == 1 and scale_b.numel() == 1:          # per-tensor: the stock kernel is already fast
        return False
    if scale_a.numel() not in (1, M) or scale_b.numel() not in (1, N):   # block-scaled schemes: stock
        return False
    if scale_a.dtype != torch.float32 or scale_b.dtype != torch.float32:
        return False
    if a.dtype != E4M3 or b.dtype != E4M3 or a.device != b.device:
        return False
    if out_dtype not in (torch.bfloat16, torch.float16):
        return False
    if bias is not None and (bias.dim() != 1 or bias.numel() != N):
        return False
    # b.t() contiguous: the common layout is read from the strides, any other through the view
    if not a.is_contiguous() or (b.stride() != (1, a.shape[1]) and not b.t().is_contiguous()) or a.shape[1] % 16 \
            or N % 16:
        return False
    if a.shape[1] == 0:                                        # an empty reduction: the stock op (the kernels refuse it)
        return False
    return True


def unit_scale(device) -> torch.Tensor:  # noqa: ANN001
    """The fp32 scalar 1.0 of a device, made once (the unit scales of the raw product)."""
    dev = torch.device(device)
    key = (dev.type, dev.index)
    one = _UNIT.get(key)
    if one is None:
        one = torch.ones((), device=dev, dtype=torch.float32)
        _UNIT[key] = one
    return one


def _vec_scales(scale_a: torch.Tensor, scale_b: torch.Tensor, M: int, N: int):
    """Per-token [M] and per-channel [N] fp32 scale vectors (scalars expanded), as the reference passes them on."""
    sa = scale_a.reshape(-1).float()
    sb = scale_b.reshape(-1).float()
    if sa.numel() == 1:
        sa = sa.expand(M)
    if sb.numel() == 1:
        sb = sb.expand(N)
    return sa.contiguous(), sb.contiguous()


def _bias(bias, out_dtype):  # noqa: ANN001,ANN202
    return bias if bias is None or bias.dtype == out_dtype else bias.to(out_dtype)


def scaled_mm_fused(a, b, scale_a, scale_b, out_dtype, bias=None):  # noqa: ANN001,ANN201
    """Kernel 2 on an eligible call (``b`` is vLLM's [K, N] view of the [N, K] weight): one launch, the scale
    epilogue on the accumulator (h3_tp2/fp8_gemm.py:240-248, fp8_cutlass.py:115-131).  The call has passed
    ``eligible``, so it takes the lean launcher (the C side re-checks sizes, strides and alignment)."""
    return ops.scaled_mm_eligible(a, b, scale_a, scale_b, out_dtype, bias)


def product_fp32(a, b) -> torch.Tensor:  # noqa: ANN001
    """The unscaled fp32 product a @ b: kernel 2's raw-accumulator mode (the reference's torch._scaled_mm with unit
    scales, h3_tp2/fp8_gemm.py:153-155, fp8_consumers.py:518-523)."""
    one = unit_scale(a.device)
    return ops.gemm(a, b.t(), one, one, torch.float32)


def _launch(x32, sa, sb, bias, y, N):  # noqa: ANN001,ANN201
    """The scale pass into ``y`` (h3_tp2/fp8_gemm.py:167-171): y = round(sa * (sb * x32)) (+ bias by one fma)."""
    del N   # the width is x32's
    return ops.scale_bias_cast(x32, sa.reshape(-1), sb.reshape(-1), _bias(bias, y.dtype), y.dtype, out=y)


def scaled_mm_tensor32(a, b, scale_a, scale_b, out_dtype, bias=None):  # noqa: ANN001,ANN201
    """The two-pass form (h3_tp2/fp8_gemm.py:149-164): fp32 product, then the scale/bias/round pass."""
    M, N = a.shape[0], b.shape[1]
    x32 = product_fp32(a, b)
    sa, sb = _vec_scales(scale_a, scale_b, M, N)
    y = torch.empty((M, N), device=a.device, dtype=out_dtype)
    return _launch(x32, sa, sb, bias, y, N)


def epilogue(acc, sa, sb, bias, out_dtype):  # noqa: ANN001,ANN201
    """The epilogue on an fp32 accumulator tensor already on the device (the scale pass kernel); the reference's
    ``epilogue_torch`` (h3_tp2/fp8_gemm.py:174-185) contract: t = sb * acc, y = sa * t or fma(sa, t, bias), one
    rounding to ``out_dtype``.  Device tensors only."""
    M, N = acc.shape
    s_a, s_b = _vec_scales(sa, sb, M, N)
    return ops.scale_bias_cast(acc, s_a, s_b, _bias(bias, out_dtype), out_dtype)


def set_stash_hook(fn) -> None:  # noqa: ANN001
    """Register a hook that may take over an eligible call and return a placeholder (fp8_swiglu: fc1 of the MLP;
    fp8_consumers: the block's qkv / out / fc2).  Hooks run in registration order after the routers."""
    with _lock:
        if fn not in _stash_hooks:
            _stash_hooks.append(fn)


def set_router(fn) -> None:  # noqa: ANN001
    """Register a router that may compute an eligible call itself (fp8_hip.route); it returns None to decline."""
    with _lock:
        if fn not in _routers:
            _routers.append(fn)


def clear_hooks() -> None:
    """Remove every router and stash hook."""
    with _lock:
        _routers.clear()
        _stash_hooks.clear()


def route(a, b, scale_a, scale_b, out_dtype, bias=None, two_pass=None):  # noqa: ANN001,ANN201
    """Dispatch of an eligible call (h3_tp2/fp8_gemm.py:328-341): routers, then stash hooks, then kernel 2 (level
    "hip") or the two-pass form ("tensor32"; ``two_pass`` replaces it, as the reference's tests pass a stand-in)."""
    for router in list(_routers):
        y = router(a, b, scale_a, scale_b, out_dtype, bias)
        if y is not None:
            _stats["routed"] += 1
            return y
    for hook in list(_stash_hooks):
        placeholder = hook(a, b, scale_a, scale_b, out_dtype, bias)
        if placeholder is not None:
            _stats["stashed"] += 1
            return placeholder
    if _state["fused"] and two_pass is None:
        _stats["hip"] += 1
        return scaled_mm_fused(a, b, scale_a, scale_b, out_dtype, bias)
    _stats["two_pass"] += 1
    return (two_pass or scaled_mm_tensor32)(a, b, scale_a, scale_b, out_dtype, bias)


def make_scaled_mm(orig):  # noqa: ANN001,ANN201
    """The replacement of ``ops.cutlass_scaled_mm``: eligible calls go to ``route``, the rest to ``orig``."""
    def _mm(a, b, scale_a, scale_b, out_dtype, bias=None):  # noqa: ANN001,ANN202
        if not eligible(a, b, scale_a, scale_b, out_dtype, bias):
            _stats["stock"] += 1
            return orig(a, b, scale_a, scale_b, out_dtype, bias)
        return route(a, b, scale_a, scale_b, out_dtype, bias)

    _mm._h3_tp2_amd = True
    _mm.__wrapped__ = orig
    return _mm


# Install-check cases: (kind, M, N, K).  The small ones run as half tiles or 128 x 192 tiles and pin the edges; the
# 4100-row ones are the serving shapes the reference checks at install (h3_tp2/fp8_cutlass.py:211-213) -- 17 token tiles
# x 21 weight tiles = 357 tiles, so they run the persistent full-tile kernel on every CU and its half-tile tail.
SELFCHECK_CASES = (("int", 200, 400, 512), ("int", 333, 272, 1024), ("int", 129, 528, 3072),
                   ("int", 4100, 5376, 1024), ("rand", 200, 1040, 2048), ("rand", 4100, 5376, 7168),
                   ("rand", 4100, 21504, 5376))


def selfcheck(device="cuda", cases=SELFCHECK_CASES) -> list[str]:  # noqa: ANN001
    """Install check on the GPU (h3_tp2/fp8_cutlass.py:204-227 plays the same part): kernel 2 against the two-pass
    form and against torch's fp32 matmul of the dequantised operands on integer-valued inputs (exact accumulators in
    any order: checks the epilogue, the tile map and the edges bit for bit), with partial row and column tiles, and the
    two forms against each other on random inputs, up to the 4100-row DiT serving shapes.  Operands are generated on
    the device.  Returns the failing cases."""
    bad = []
    g = torch.Generator(device=device).manual_seed(0)
    for kind, M, N, K in cases:
        if kind == "int":
            a = torch.randint(-4, 5, (M, K), generator=g, device=device).float()
            w = torch.randint(-2, 3, (N, K), generator=g, device=device).float()
        else:
            a = (torch.randn(M, K, generator=g, device=device) * 64).clamp(-448, 448)
            w = (torch.randn(N, K, generator=g, device=device) * 64).clamp(-448, 448)
        sa = torch.exp(torch.empty(M, 1, device=device).uniform_(-9.0, -2.0, generator=g))
        sb = torch.exp(torch.empty(N, device=device).uniform_(-9.5, -7.5, generator=g))
        ad, wd = a.to(E4M3), w.to(E4M3)
        del a, w
        y = scaled_mm_fused(ad, wd.t(), sa, sb, torch.bfloat16)
        y2 = scaled_mm_tensor32(ad, wd.t(), sa, sb, torch.bfloat16)
        ok = torch.equal(y.view(torch.int16), y2.view(torch.int16))
        if kind == "int":
            acc = ad.float() @ wd.float().t()                      # exact: |acc| <= 8 K < 2^24
            ref = ((sb.view(1, -1) * acc) * sa.view(-1, 1)).to(torch.bfloat16)
            ok = ok and torch.equal(y.view(torch.int16), ref.view(torch.int16))
        if not ok:
            bad.append(f"{kind} M={M} N={N} K={K}")
        del ad, wd, y, y2
    torch.cuda.synchronize(device)
    return bad


def install(ops_module=None, level: str = "hip", check: bool = True) -> bool:  # noqa: ANN001
    """Replace ``ops_module.cutlass_scaled_mm`` (vLLM's ``_custom_ops`` by default) with the dispatcher at ``level``.

    The library is loaded first (a missing or mismatched libh3fp8 raises: there is no silent fallback for a requested
    level).  With ``check`` the install check runs on the GPU; if it fails nothing is replaced, the stock op stays and
    False is returned (the reference likewise keeps a working path when a level's probe fails,
    h3_tp2/fp8_gemm.py:387-410).  Level "off" leaves the op alone."""
    if level not in LEVELS:
        raise ValueError(f"FP8 GEMM level must be one of {sorted(LEVELS)}, got {level!r}")
    if ops_module is None:
        from vllm import _custom_ops as ops_module  # noqa: PLC0415  (the caller passes the module where vLLM is absent)
    orig = ops_module.cutlass_scaled_mm
    if getattr(orig, "_h3_tp2_amd", False):
        return True
    if level == "off":
        _state.update(level="off", fused=False)
        return False
    _lib.load()
    if check:
        try:
            bad = selfcheck()
        except Exception as exc:  # noqa: BLE001
            bad = [f"{type(exc).__name__}: {exc}"]
        _state["selfcheck"] = bad
        if bad:
            logger.warning("h3_tp2_amd: FP8 GEMM install check failed (%s); the stock op stays", "; ".join(bad))
            return False
    ops_module.cutlass_scaled_mm = make_scaled_mm(orig)
    _state.update(level=level, fused=level == "hip", triton=True, installed=True)
    logger.warning("h3_tp2_amd: FP8 GEMM dispatcher ON, level %s (%s)", level,
                   "gfx950 kernel 2, scale epilogue in registers" if level == "hip"
                   else "raw fp32 product + device scale pass")
    return True


def stats() -> dict:
    return dict(_stats)
