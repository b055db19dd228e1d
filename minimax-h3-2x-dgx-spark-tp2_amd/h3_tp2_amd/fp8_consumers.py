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
fp32 product to stash: the hook stands down and the consumers read kernel 2's bf16 output.  That is also the level
that moves the fewest bytes on MI355X (2 B written + 2 B read per output element, against 4 + 4 for the fp32
product), so the fused consumers below serve the two-pass level.

The fused consumers (``qk_norm_rope_fused``, ``gate_rms_fused``, ``gate_fused``, the reference's :424-504 launchers)
read the fp32 product through the scale pass's epilogue and its one rounding to bf16, then run the stock consumer's
arithmetic (``h3fp8_scale_qk_norm_rope``, ``h3fp8_scale_gate_rms_quant``, ``h3fp8_scale_indexed_gate``).  ``install``
registers them per site (``set_fused``) behind the reference's checks -- ``qk_mismatch`` / ``rows_mismatch``
(:590-637) and a bit-for-bit self-check against the scale pass + the stock consumer on the first 64 rows once per
(site, shape) (:560-580), whose failure disables the site.  Their sums of squares are rounded once from an exact
(fp64) sum: a stock consumer whose fp32 reduction rounds differently fails the self-check on some rows and the site
then stays stock.
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
HEAD_DIM = 128
ROTARY_DIM = 96
_SELFCHECK_ROWS = 64

_tls = threading.local()   # ctx: the _Ctx of the DiT block whose forward is running in this thread
_state: dict[str, Any] = {"sites": (), "disabled": set(), "fused": {}, "checked": {}}
_stats = {"stash": 0, "fused": 0, "materialize": 0, "stock": 0, "fused_qkv": 0, "fused_out": 0, "fused_fc2": 0,
          "selfcheck_pass": 0, "selfcheck_fail": 0}
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


# ---- the fused consumers on an explicit stash ----------------------------------------------------------------------

def qk_norm_rope_fused(st: Stash, num_heads: int, num_kv_heads: int, head_dim: int, q_weight: torch.Tensor,
                       k_weight: torch.Tensor, rope_table: torch.Tensor, eps: float):
    """q, k = ``fused_qk_norm_rope`` of the qkv GEMM output read from the fp32 product; v's columns are scale-passed
    into the placeholder ``st.ph`` (so ``ph[:, q+k:]`` viewed [T, kv_heads, d] is the stock v).  Returns (q, k, v)."""
    from . import ops
    x32, sa, sb, bias, ph = st.x32, st.sa, st.sb, st.bias, st.ph
    T = x32.shape[0]
    v0 = (num_heads + num_kv_heads) * head_dim
    oq, ok = ops.scale_qk_norm_rope(x32, sa, sb, bias, num_heads, num_kv_heads, q_weight.contiguous(),
                                    k_weight.contiguous(), rope_table, eps)
    if T:
        ops.scale_bias_cast(x32[:, v0:], sa, sb[v0:], None if bias is None else bias[v0:], torch.bfloat16,
                            out=ph[:, v0:])
    return oq, ok, ph[:, v0:].view(T, num_kv_heads, head_dim)


def gate_rms_fused(st: Stash, residual: torch.Tensor, gate: torch.Tensor, weight: torch.Tensor, shift: torch.Tensor,
                   scale: torch.Tensor, indices: torch.Tensor, eps: float, reuse_placeholder: bool = True):
    """``indexed_gate_rms_norm_scale_shift(residual, gate, branch, ...)`` with branch = the out projection's output
    read from the fp32 product; residual_out goes into the placeholder (the stock ``empty_like(residual)`` layout)."""
    from . import ops
    out = st.ph if reuse_placeholder else None
    return ops.scale_gate_rms_quant(st.x32, st.sa, st.sb, st.bias, residual, gate, weight, shift, scale, indices, eps,
                                    residual_out=out)


def gate_fused(st: Stash, x: torch.Tensor, gate: torch.Tensor, indices: torch.Tensor,
               reuse_placeholder: bool = True) -> torch.Tensor:
    """``indexed_gate(x, gate, other, indices)`` with other = the fc2 output read from the fp32 product; the result
    goes into the placeholder when ``x`` is contiguous (the stock ``empty_like(x)``)."""
    from . import ops
    out = st.ph if (reuse_placeholder and x.is_contiguous()) else None
    return ops.scale_indexed_gate(st.x32, st.sa, st.sb, st.bias, x, gate, indices, out=out)


def _bits(t: torch.Tensor) -> torch.Tensor:
    t = t.contiguous()
    return t.view({1: torch.uint8, 2: torch.int16, 4: torch.int32}[t.element_size()])


def _selfcheck(key, fused_fn, stock_fn) -> bool:  # noqa: ANN001
    """Once per (site, shape): fused vs the scale pass + stock consumer on the first rows, bit for bit; a mismatch (or
    an exception) disables the site for the process."""
    ok = _state["checked"].get(key)
    if ok is not None:
        return ok
    try:
        fused, stock = fused_fn(), stock_fn()
        ok = len(fused) == len(stock) and all(
            f.shape == s.shape and f.dtype == s.dtype and torch.equal(_bits(f), _bits(s)) for f, s in zip(fused, stock))
    except Exception as exc:  # noqa: BLE001
        logger.warning("h3_tp2_amd fp8 consumers: self-check %s raised %s: %s", key, type(exc).__name__, exc)
        ok = False
    _state["checked"][key] = ok
    if ok:
        _stats["selfcheck_pass"] += 1
    else:
        _stats["selfcheck_fail"] += 1
        _state["disabled"].add(key[0])
        logger.warning("h3_tp2_amd fp8 consumers: self-check %s not bit-identical to the scale pass + the stock "
                       "consumer; site %s disabled", key, key[0])
    return ok


def _on_gpu(*ts: torch.Tensor) -> bool:
    dev = ts[0].device
    return dev.type == "cuda" and all(isinstance(t, torch.Tensor) and t.device == dev for t in ts)


def qk_mismatch(st: Stash, q, k, q_weight, k_weight, rope_table, head_dim, rotary_dim, interleaved) -> str | None:  # noqa: ANN001
    """None when (q, k) are exactly the q/k views of the stash's placeholder and the kernel takes the call
    (half-split, head_dim 128, rotary 96), else the reason."""
    ph = st.ph
    if interleaved:
        return "interleaved"
    if q.dim() != 3 or k.dim() != 3 or q.dtype != torch.bfloat16 or k.dtype != torch.bfloat16:
        return "q/k rank or dtype"
    T, H, D = q.shape
    Hk = k.shape[1]
    N = ph.shape[1]
    if T == 0 or ph.dim() != 2 or ph.shape[0] != T or k.shape != (T, Hk, D) or N != (H + 2 * Hk) * D:
        return "shapes"
    if not ph.is_contiguous() or not st.x32.is_contiguous() or st.x32.shape != ph.shape:
        return "placeholder/product layout"
    eq, ek = ph[:, :H * D].view(T, H, D), ph[:, H * D:(H + Hk) * D].view(T, Hk, D)
    if q.data_ptr() != eq.data_ptr() or k.data_ptr() != ek.data_ptr() or q.stride() != eq.stride() \
            or k.stride() != ek.stride():
        return "q/k are not the split views of the qkv placeholder"
    if D != HEAD_DIM or head_dim not in (None, D):
        return "head_dim"
    rot = rope_table.shape[-1] if rope_table.dim() == 2 else -1
    if rot != ROTARY_DIM or rotary_dim not in (None, rot) or rope_table.shape != (T, rot) or rope_table.stride(1) != 1:
        return "rotary"
    if rope_table.dtype not in (torch.bfloat16, torch.float32) or q_weight.shape != (D,) or k_weight.shape != (D,) \
            or q_weight.dtype != torch.bfloat16 or k_weight.dtype != torch.bfloat16:
        return "rope table or norm weight dtype/shape"
    if not _on_gpu(st.x32, q_weight, k_weight, rope_table):
        return "device"
    return None


def rows_mismatch(st: Stash, x: torch.Tensor, branch: torch.Tensor, *others: torch.Tensor) -> str | None:
    """None when ``branch`` is exactly the stash's placeholder and ``x`` (the residual) a contiguous bf16 tensor of the
    same shape on the same device as the other operands (gate / shift / scale rows, then the indices)."""
    ph = st.ph
    if branch.data_ptr() != ph.data_ptr() or branch.shape != ph.shape or branch.stride() != ph.stride():
        return "branch is not the placeholder"
    if x.dim() != 2 or x.shape != ph.shape or x.dtype != torch.bfloat16 or not x.is_contiguous() \
            or not ph.is_contiguous() or not st.x32.is_contiguous() or st.x32.shape != ph.shape:
        return "residual shape/dtype/layout"
    if x.shape[0] == 0:
        return "no rows"
    H = x.shape[1]
    if H % 8 or H > 8192:
        return "width"
    for o in others[:-1]:
        if o.dim() != 2 or o.stride(1) != 1 or o.dtype != torch.bfloat16 or o.shape[1] != H or o.shape[0] == 0 \
                or (o.shape[0] > 1 and o.stride(0) % 8) or o.data_ptr() % 16:
            return "gate/shift/scale layout"
    idx = others[-1]
    if idx.dim() != 1 or idx.shape[0] != x.shape[0] or idx.dtype not in (torch.int32, torch.int64):
        return "indices"
    if not _on_gpu(x, st.x32, *others):
        return "device"
    return None


def make_fused_qk(orig):  # noqa: ANN001,ANN201
    """The qkv site's fused consumer (registered by ``install``): ``fused_qk_norm_rope``'s arguments after the stash."""
    def fused(st, q, k, q_weight, k_weight, rope_table, eps, *, head_dim=None, rotary_dim=None, interleaved=False):  # noqa: ANN001,ANN202
        reason = qk_mismatch(st, q, k, q_weight, k_weight, rope_table, head_dim, rotary_dim, interleaved)
        if reason is not None:
            _warn_once("qkv-" + reason, "qkv consumer not fused (%s)", reason)
            return None
        H, Hk, D = q.shape[1], k.shape[1], q.shape[-1]
        r = min(_SELFCHECK_ROWS, q.shape[0])

        def _fused_sub():  # noqa: ANN202
            return qk_norm_rope_fused(st.rows(r), H, Hk, D, q_weight, k_weight, rope_table[:r], eps)

        def _stock_sub():  # noqa: ANN202
            p = st.rows(r).materialize()
            oq, ok_ = orig(p[:, :H * D].view(r, H, D), p[:, H * D:(H + Hk) * D].view(r, Hk, D), q_weight, k_weight,
                           rope_table[:r], eps, head_dim=head_dim, rotary_dim=rotary_dim, interleaved=interleaved)
            return oq, ok_, p[:, (H + Hk) * D:].view(r, Hk, D)

        if not _selfcheck(("qkv", tuple(st.ph.shape[1:]), rope_table.dtype), _fused_sub, _stock_sub):
            return None
        out_q, out_k, _ = qk_norm_rope_fused(st, H, Hk, D, q_weight, k_weight, rope_table, eps)
        _stats["fused_qkv"] += 1
        return out_q, out_k

    return fused


def make_fused_gate_rms(orig):  # noqa: ANN001,ANN201
    """The out site's fused consumer: ``indexed_gate_rms_norm_scale_shift``'s arguments after the stash."""
    def fused(st, residual, gate, branch, weight, shift, scale, indices, eps):  # noqa: ANN001,ANN202
        reason = rows_mismatch(st, residual, branch, gate, shift, scale, indices)
        if reason is None and (weight.shape != (residual.shape[1],) or weight.dtype != torch.bfloat16
                               or not weight.is_contiguous() or weight.device != residual.device
                               or weight.data_ptr() % 16):
            reason = "norm weight"
        if reason is not None:
            _warn_once("out-" + reason, "out consumer not fused (%s)", reason)
            return None
        r = min(_SELFCHECK_ROWS, residual.shape[0])

        def _fused_sub():  # noqa: ANN202
            return gate_rms_fused(st.rows(r), residual[:r], gate, weight, shift, scale, indices[:r], eps)

        def _stock_sub():  # noqa: ANN202
            p = st.rows(r).materialize()
            return orig(residual[:r], gate, p, weight, shift, scale, indices[:r], eps)

        if not _selfcheck(("out", tuple(residual.shape[1:]), gate.dtype, weight.dtype), _fused_sub, _stock_sub):
            return None
        res = gate_rms_fused(st, residual, gate, weight, shift, scale, indices, eps)
        _stats["fused_out"] += 1
        return res

    return fused


def make_fused_gate(orig):  # noqa: ANN001,ANN201
    """The fc2 site's fused consumer: ``indexed_gate``'s arguments after the stash."""
    def fused(st, x, gate, other, indices):  # noqa: ANN001,ANN202
        reason = rows_mismatch(st, x, other, gate, indices)
        if reason is not None:
            _warn_once("fc2-" + reason, "fc2 consumer not fused (%s)", reason)
            return None
        r = min(_SELFCHECK_ROWS, x.shape[0])

        def _fused_sub():  # noqa: ANN202
            return (gate_fused(st.rows(r), x[:r].contiguous(), gate, indices[:r], reuse_placeholder=False),)

        def _stock_sub():  # noqa: ANN202
            p = st.rows(r).materialize()
            return (orig(x[:r].contiguous(), gate, p, indices[:r]),)

        if not _selfcheck(("fc2", tuple(x.shape[1:]), gate.dtype), _fused_sub, _stock_sub):
            return None
        out = gate_fused(st, x, gate, indices)
        _stats["fused_fc2"] += 1
        return out

    return fused


FUSED_FACTORIES = {"qkv": make_fused_qk, "out": make_fused_gate_rms, "fc2": make_fused_gate}


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


def install(sites=SITES, tr=None, *, lora_types=None, fused: bool = True) -> list[str]:  # noqa: ANN001
    """Wrap the block forward and the sites' consumers in the transformer module ``tr`` and register the stash hook;
    with ``fused`` also the fused consumer kernels of the sites.  Needs the dispatcher's two-pass level (at the
    default level there is no fp32 product to stash)."""
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
        orig = getattr(tr, name)
        setattr(tr, name, make_consumer_wrapper(site, orig))
        if fused:
            set_fused(site, FUSED_FACTORIES[site](orig))
    block_cls.forward = make_block_forward(block_cls.forward, sites, lora_types)
    fp8_gemm.set_stash_hook(stash_hook)
    _state["sites"] = sites
    return list(sites)


def stats() -> dict:
    return dict(_stats)
