"""The GEMM-output stash protocol of the DiT block on MI355X (the consumer side of the dispatcher's stash hooks).

Mirrors the reference's h3_tp2/fp8_consumers.py protocol -- ``Stash`` (:388-399), ``scale_pass_into`` (:373-380),
``_product_fp32`` (:518-523), ``_vec`` (:526-528), ``stash_hook`` (:531-546), ``_materialize_all`` (:549-555),
``_take`` (:640-648), the consumer wrappers (:651-747), ``block_plan`` (:758-784), ``make_block_forward`` (:787-808),
``parse_sites`` (:811-819), ``install`` (:859-916) -- on the HIP kernels:

* at the dispatcher's two-pass level ("tensor32"), a GEMM on the qkv / out / fc2 weight of the running block keeps its
  fp32 product (kernel 2, raw-accumulator mode) and its epilogue operands in a ``Stash``; the layer receives an
  uninitialised bf16 placeholder;
* the block's consumer of that output (``fused_qk_norm_rope``, ``indexed_gate_rms_norm_scale_shift``,
  ``indexed_gate``) takes the stash: with a fused consumer registered for the site it reads the product directly;
  otherwise, and on any mismatch of pointer, shape or flags, the stash is materialised -- the scale pass
  (``h3fp8_scale_bias_cast``: t = sb * acc, y = sa * t or fma(sa, t, bias), one rounding to bf16) writes the
  placeholder -- and the stock consumer runs, so the fallback is the stock path bit for bit.

At the dispatcher's default level ("hip", one kernel-2 launch per GEMM with the epilogue in registers) there is no
fp32 product to stash: the hook stands down and the consumers read kernel 2's bf16 output.  Fused consumer kernels
(the qk-RMSNorm + RoPE and gate-residual RMS/AdaLN kernels reading the accumulator) are registered per site through
``set_fused``; none ships in this library yet.
"""
from __future__ import annotations

import functools
import logging
import threading
from typing import Any, Callable

import torch

from . import fp8_gemm

logger = logging.getLogger("h3_tp2_amd.fp8_consumers")

SITES = ("qkv", "out", "fc2")
CONSUMERS = {"qkv": "fused_qk_norm_rope", "out": "indexed_gate_rms_norm_scale_shift", "fc2": "indexed_gate"}

_tls = threading.local()   # ctx: the _Ctx of the DiT block whose forward is running in this thread
_state: dict[str, Any] = {"sites": (), "disabled": set(), "fused": {}}
_stats = {"stash": 0, "fused": 0, "materialize": 0, "stock": 0}
_warned: set = set()


def _warn_once(key: str, msg: str, *args: Any) -> None:
    if key not in _warned:
        _warned.add(key)
        logger.warning("h3_tp2_amd fp8 consumers: " + msg, *args)


def scale_pass_into(x32: torch.Tensor, sa: torch.Tensor, sb: torch.Tensor, bias: torch.Tensor | None,
                    y: torch.Tensor) -> torch.Tensor:
    """The ordinary scale pass into ``y`` (the stock output of the two-pass GEMM), on the device."""
    return fp8_gemm._launch(x32, sa, sb, bias, y, x32.shape[1])


class Stash:
    """The fp32 product of one GEMM and its epilogue operands, kept in place of the scale pass's output ``ph``."""
    __slots__ = ("x32", "sa", "sb", "bias", "ph")

    def __init__(self, x32: torch.Tensor, sa: torch.Tensor, sb: torch.Tensor, bias: torch.Tensor | None,
                 ph: torch.Tensor):
        self.x32, self.sa, self.sb, self.bias, self.ph = x32, sa, sb, bias, ph

    def materialize(self) -> torch.Tensor:
        return scale_pass_into(self.x32, self.sa, self.sb, self.bias, self.ph)

    def rows(self, r: int) -> "Stash":
        return Stash(self.x32[:r], self.sa[:r], self.sb, self.bias, torch.empty_like(self.ph[:r]))


class _Ctx:
    __slots__ = ("want", "pending")

    def __init__(self, want: dict):
        self.want = want          # (weight data_ptr, weight shape) -> site
        self.pending: dict[str, Stash] = {}


def _vec(scale: torch.Tensor, n: int) -> torch.Tensor:
    s = scale.reshape(-1).float()
    return (s.expand(n) if s.numel() == 1 else s).contiguous()


def stash_hook(a, b, scale_a, scale_b, out_dtype, bias):  # noqa: ANN001
    """Dispatcher stash hook: when ``b`` is the qkv / out / fc2 weight of the running block (and the dispatcher runs
    the two-pass level), keep the fp32 product and return an uninitialised placeholder."""
    ctx = getattr(_tls, "ctx", None)
    if ctx is None or out_dtype is not torch.bfloat16 or fp8_gemm._state.get("fused"):
        return None
    site = ctx.want.pop((b.data_ptr(), tuple(b.shape)), None)
    if site is None:
        return None
    if ctx.pending:                       # a stash that was never consumed: make it real before the next one
        _materialize_all(ctx, f"unconsumed stash before {site}")
    M, N = a.shape[0], b.shape[1]
    ph = torch.empty((M, N), device=a.device, dtype=out_dtype)
    ctx.pending[site] = Stash(fp8_gemm.product_fp32(a, b), _vec(scale_a, M), _vec(scale_b, N), bias, ph)
    _stats["stash"] += 1
    return ph


def _materialize_all(ctx: _Ctx, reason: str) -> None:
    for site, st in list(ctx.pending.items()):
        st.materialize()
        _stats["materialize"] += 1
        _warn_once("mat-" + reason, "%s: stash of %s materialised, stock consumer", reason, site)
    ctx.pending.clear()


def _take(site: str):  # noqa: ANN202
    """(ctx, the site's stash or None); another site's pending stash is materialised first."""
    ctx = getattr(_tls, "ctx", None)
    if ctx is None or not ctx.pending:
        return ctx, None
    st = ctx.pending.get(site)
    if st is None:
        _materialize_all(ctx, f"{site} consumer saw another site's stash")
    return ctx, st


def set_fused(site: str, fn: Callable | None) -> None:
    """Register the fused consumer of ``site``: ``fn(stash, *args, **kwargs)`` returns the consumer's result computed
    from the stash, or None when it cannot take the call (the stash is then materialised and the stock consumer
    runs).  ``None`` removes it."""
    if site not in SITES:
        raise ValueError(f"unknown consumer site {site!r}")
    if fn is None:
        _state["fused"].pop(site, None)
    else:
        _state["fused"][site] = fn


def make_consumer_wrapper(site: str, orig):  # noqa: ANN001,ANN201
    """The wrapper of a site's consumer: the fused consumer on the site's stash when one is registered and takes the
    call, otherwise the stash materialised and the stock consumer."""
    @functools.wraps(orig)
    def consumer(*args, **kwargs):  # noqa: ANN002,ANN003,ANN202
        ctx, st = _take(site)
        if st is not None:
            fn = _state["fused"].get(site)
            if fn is not None and site not in _state["disabled"]:
                out = fn(st, *args, **kwargs)
                if out is not None:
                    del ctx.pending[site]
                    _stats["fused"] += 1
                    return out
            _materialize_all(ctx, f"{site}: no fused consumer took the call")
            _stats["stock"] += 1
        return orig(*args, **kwargs)

    consumer._h3_tp2_amd_consumer = True
    return consumer


def block_plan(block, sites, lora_types=()) -> tuple[dict | None, str]:  # noqa: ANN001
    """{(weight data_ptr, weight shape): site} for this block's eligible GEMMs, or (None, reason)."""
    try:
        if torch.compiler.is_compiling():
            return None, "torch.compile tracing"
    except AttributeError:
        pass
    layers = {"qkv": getattr(getattr(block, "attn", None), "qkv_proj", None),
              "out": getattr(getattr(block, "attn", None), "out_proj", None),
              "fc2": getattr(getattr(block, "mlp", None), "fc2", None)}
    want: dict = {}
    for site in sites:
        if site in _state["disabled"]:
            continue
        layer = layers[site]
        if layer is None or (lora_types and isinstance(layer, lora_types)):
            return None, f"{site}: missing or LoRA-wrapped layer"
        if getattr(layer, "tp_size", 1) != 1:
            return None, f"{site}: tp_size != 1 (an all-reduce would read the placeholder)"
        w = getattr(layer, "weight", None)
        n = int(getattr(layer, "output_size_per_partition", 0) or 0)
        if not isinstance(w, torch.Tensor) or w.dtype != torch.float8_e4m3fn or w.dim() != 2 or w.shape[1] != n:
            return None, f"{site}: weight is not an unpadded FP8 [K, N] tensor"
        want[(w.data_ptr(), tuple(w.shape))] = site
    return (want or None), "no site left"


def make_block_forward(orig_forward, sites, lora_types=()):  # noqa: ANN001,ANN201
    @functools.wraps(orig_forward)
    def forward(self, *args, **kwargs):  # noqa: ANN001,ANN202
        want, reason = block_plan(self, sites, lora_types)
        if want is None:
            _warn_once("plan-" + reason, "block not planned (%s); stock path", reason)
            return orig_forward(self, *args, **kwargs)
        prev = getattr(_tls, "ctx", None)
        ctx = _Ctx(want)
        _tls.ctx = ctx
        ok = False
        try:
            out = orig_forward(self, *args, **kwargs)
            ok = True
            return out
        finally:
            _tls.ctx = prev
            if ctx.pending:
                if ok:
                    _materialize_all(ctx, "stash left at the end of the block")
                ctx.pending.clear()

    forward._h3_tp2_amd_consumer = True
    return forward


def parse_sites(value: str | None) -> tuple[str, ...]:
    """"1"/"all" = every site; a comma list of qkv,out,fc2; empty/"0"/"off" = none."""
    v = (value or "").strip().lower()
    if v in ("1", "all", "on", "true"):
        return SITES
    if not v or v in ("0", "off", "false"):
        return ()
    return tuple(s for s in SITES if s in {p.strip() for p in v.split(",")})


def install(sites=SITES, tr=None, *, lora_types=None) -> list[str]:  # noqa: ANN001
    """Wrap the block forward and the sites' consumers in the transformer module ``tr`` and register the stash hook.
    Needs the dispatcher's two-pass level (at the default level there is no fp32 product to stash)."""
    sites = tuple(s for s in SITES if s in sites)
    if not sites:
        return []
    if fp8_gemm._state.get("level") != "tensor32" or fp8_gemm._state.get("fused"):
        logger.warning("h3_tp2_amd fp8 consumers: needs the dispatcher's two-pass level; skipped")
        return []
    if tr is None:
        from vllm_omni.diffusion.models.minimax_h3 import minimax_h3_transformer as tr  # noqa: PLC0415
    if lora_types is None:
        try:
            from vllm.lora.layers import BaseLayerWithLoRA  # noqa: PLC0415
            lora_types = (BaseLayerWithLoRA,)
        except ImportError:
            lora_types = ()
    block_cls = tr.MiniMaxH3DiTBlock
    if getattr(block_cls.forward, "_h3_tp2_amd_consumer", False):
        return list(_state["sites"])
    for site in sites:
        name = CONSUMERS[site]
        setattr(tr, name, make_consumer_wrapper(site, getattr(tr, name)))
    block_cls.forward = make_block_forward(block_cls.forward, sites, lora_types)
    fp8_gemm.set_stash_hook(stash_hook)
    _state["sites"] = sites
    return list(sites)


def stats() -> dict:
    return dict(_stats)
