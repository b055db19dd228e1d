"""Per-token dynamic FP8 activation quant on MI355X: the drop-in for ``QuantFP8.forward`` and the producer-fused
quant protocol.

Mirrors the reference's h3_tp2/fp8_quant_fuse.py host surface -- ``quant`` (:318-327), ``rms_quant`` (:330-346),
``gate_rms_quant`` (:349-369), ``unpack_stock`` / ``unpack_quant`` (:372-385), ``silu_mul_quant`` (:392-402),
``Pending`` (:432-450), ``_Ctx`` (:453-459), ``_selfcheck`` / ``_pick_mode`` (:477-511), ``make_quant_forward`` (:553-576), ``_layer_post_hook`` (:579-588),
``_quant_of`` (:591-603), ``block_plan`` (:614-645), ``make_block_forward`` (:648-670), ``_take_site`` (:673-680),
``_rows_ok`` (:691-693), ``make_rms_wrapper`` (:702-736), ``make_gate_rms_wrapper`` (:739-779), ``make_act_forward``
(:806-828), ``parse_sites`` (:836-844), ``install`` (:925-1003) -- with the compute on kernel 1, the producer kernels
and the SwiGLU + quant kernel:

* ``QuantFP8.forward`` of a dynamic per-token instance on a bf16 [M, K] input runs kernel 1 (one wavefront per row:
  amax = max_k |x_k| NaN-propagating, scale = max(amax / 448, 1/(448*512)), q = e4m3fn_rne(clamp(x * (1/scale),
  +-448))), unless a producer already left that layer's (fp8, scale) pending, which is then returned as is;
* the fc2 site: the MLP's ``SiluAndMul`` on fc1's bf16 output computes silu(gate) * up and its per-token quant in one
  pass and leaves them pending for fc2's quant; the layer holds an uninitialised bf16 placeholder.  A stash that is
  not consumed by exactly its planned quant (instance, data pointer, shape, strides, no static scale) is
  materialised first -- the stock producer is run into the placeholder -- so the fallback is the stock path;
* the qkv / fc1 sites: ``rms_norm_indexed_scale_shift`` (the block's norm1 before the QKV projection) and
  ``indexed_gate_rms_norm_scale_shift`` (the gated residual + norm2 before fc1) write the e4m3 row and its scale
  instead of the bf16 row (mode 0, the placeholder stays uninitialised) or as well as it (mode 1).  The first call per
  (site, width) runs both modes' self-check against the stock producer + the layer's own quant on the first rows, bit
  for bit; a site with no bit-identical mode is disabled for the process.

The producer kernels sum the squares exactly (fp64, one rounding to fp32); a stock producer whose fp32 reduction
rounds differently fails the self-check on some rows and its site stays stock.  ``own_producers=True`` (env
``H3_TP2_AMD_OWN_PRODUCERS=1``) also replaces the stock producers by the same kernels without the quant, so the fused
and the stock forms agree by construction.  The out site (the Ulysses reverse exchange's unpack) exists only with
sequence parallelism across GPUs; ``unpack_quant`` is its kernel (the receive buffer read in place), but ``install``
skips the site with a warning: its hook lives in the multi-GPU exchange, which this single-GPU build does not carry.
"""
from __future__ import annotations

import functools
import logging
import os
import threading
from typing import Any, Callable

import torch

from . import ops

logger = logging.getLogger("h3_tp2_amd.fp8_quant_fuse")

E4M3 = torch.float8_e4m3fn
FP8_MAX = ops.FP8_MAX
MIN_SCALE = ops.MIN_SCALE
SITES = ("qkv", "out", "fc1", "fc2")
WIRED_SITES = ("qkv", "fc1", "fc2")
_SELFCHECK_ROWS = 64

_tls = threading.local()   # ctx: _Ctx of the DiT block whose forward is running in this thread
_state: dict[str, Any] = {"sites": (), "checked": {}, "disabled": set(), "orig_quant": None, "quant_cls": None,
                          "act_cls": None, "kernel1": False, "verify": False, "modes": (0, 1), "own_producers": False}
_stats: dict[str, int] = {"kernel1": 0, "stock_quant": 0, "fused_qkv": 0, "fused_fc1": 0, "fused_fc2": 0,
                          "consumed": 0, "materialize": 0, "rerun": 0, "selfcheck_pass": 0, "selfcheck_fail": 0,
                          "verify_calls": 0, "verify_mismatch": 0, "own_producer": 0}
_warned: set = set()


def _warn_once(key: str, msg: str, *args: Any) -> None:
    if key not in _warned:
        _warned.add(key)
        logger.warning("h3_tp2_amd fp8 quant: " + msg, *args)


# ---- the kernels ----------------------------------------------------------------------------------------------------

def quant(h: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Kernel 1 on a bf16 [M, K] tensor: (fp8 [M, K], fp32 scale [M, 1])."""
    return ops.quant_rows(h)


def rms_quant(x, weight, shift, scale, indices, eps, stock=None, ph=None):  # noqa: ANN001,ANN201
    """``rms_norm_indexed_scale_shift`` + the per-token quant of its output: (fp8 [M, H], scale [M, 1]).  With ``ph``
    (bf16, like ``x``) the modulated bf16 row is stored there too.  ``stock`` is accepted for the reference's
    signature; the kernel runs on the GPU only."""
    return ops.rms_quant(x, weight, shift, scale, indices, eps, ph)


def gate_rms_quant(residual, gate, branch, weight, shift, scale, indices, eps, stock=None, ph=None):  # noqa: ANN001,ANN201
    """``indexed_gate_rms_norm_scale_shift`` with the modulated output quantised per token: (residual_out bf16 [M, H],
    fp8 [M, H], scale [M, 1]); ``ph`` as in ``rms_quant``."""
    return ops.gate_rms_quant(residual, gate, branch, weight, shift, scale, indices, eps, ph)


def unpack_stock(recv: torch.Tensor, heads: int) -> torch.Tensor:
    """The Ulysses reverse exchange's unpack: receive [P, M, hl, d] -> [1, M, heads, d] contiguous (torch copy)."""
    ws, m, hl, d = recv.shape
    result = torch.empty((1, m, heads, d), dtype=recv.dtype, device=recv.device)
    result[0].view(m, ws, hl, d).copy_(recv.transpose(0, 1))
    return result


def unpack_quant(recv: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """The unpack + the per-token quant of the [M, P*hl*d] out-projection input, read straight from the receive buffer
    [P, M, hl, d] (kernel 1 on P segments): (fp8 [M, P*hl*d], scale [M, 1])."""
    return ops.quant_from_recv(recv)


def silu_mul_quant(x: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """silu(x[:, :d]) * x[:, d:] on bf16 [M, 2d] (each product rounded to bf16) + the per-token quant of the [M, d]
    result: (fp8 [M, d], fp32 scale [M, 1])."""
    return ops.silu_mul_quant(x)


# ---- the QuantFP8 drop-in -------------------------------------------------------------------------------------------

def dynamic_per_token(quant_obj) -> bool:  # noqa: ANN001
    """True for a ``QuantFP8`` instance that computes a dynamic per-token scale (the only form kernel 1 replaces):
    not static, per token, no group quant, no token padding (the attribute checks of fp8_quant_fuse.py:596-600)."""
    return (not getattr(quant_obj, "static", True) and getattr(quant_obj, "use_per_token_if_dynamic", False)
            and not getattr(quant_obj, "is_group_quant", True) and getattr(quant_obj, "num_token_padding", 0) is None)


def kernel1_takes(x) -> bool:  # noqa: ANN001
    """Inputs kernel 1 takes: a bf16 CUDA tensor of 2 dims with contiguous rows, K % 8 == 0, 16-byte aligned rows."""
    return (isinstance(x, torch.Tensor) and x.is_cuda and x.dtype == torch.bfloat16 and x.dim() == 2
            and (x.shape[1] <= 1 or x.stride(1) == 1) and x.shape[1] % 8 == 0
            and (x.shape[0] <= 1 or x.stride(0) % 8 == 0) and x.data_ptr() % 16 == 0)


class Pending:
    """A producer's (fp8, scale) waiting for the quant of ``layer``; ``ph`` is the bf16 placeholder the model holds and
    ``k`` the GEMM input width (the quant sees ``ph`` as a contiguous [numel / k, k] view)."""
    __slots__ = ("site", "ph", "k", "q", "scale", "quant", "layer", "fill")

    def __init__(self, site: str, ph: torch.Tensor, k: int, q: torch.Tensor, scale: torch.Tensor, quant_obj,  # noqa: ANN001
                 layer, fill: Callable[[torch.Tensor], None]):
        self.site, self.ph, self.k, self.q, self.scale = site, ph, k, q, scale
        self.quant, self.layer, self.fill = quant_obj, layer, fill

    def matches(self, quant_obj, x) -> bool:  # noqa: ANN001
        ph, k = self.ph, self.k
        return (quant_obj is self.quant and isinstance(x, torch.Tensor) and x.dim() == 2 and x.dtype == ph.dtype
                and x.device == ph.device and x.data_ptr() == ph.data_ptr()
                and tuple(x.shape) == (ph.numel() // k, k) and x.stride() == (k, 1) and ph.is_contiguous())

    def materialize(self) -> torch.Tensor:
        self.fill(self.ph)        # the stock producer's bf16 output into the placeholder
        return self.ph


class _Ctx:
    __slots__ = ("block", "plan", "pending")

    def __init__(self, block, plan: dict):  # noqa: ANN001
        self.block = block
        self.plan = plan            # site -> (layer, its QuantFP8 instance)
        self.pending: Pending | None = None


def _materialize(ctx: _Ctx, reason: str) -> None:
    p = ctx.pending
    if p is None:
        return
    ctx.pending = None
    p.materialize()
    _stats["materialize"] += 1
    _warn_once("mat-" + reason, "%s: %s stash materialised (stock producer into the placeholder)", reason, p.site)


def _bits(t: torch.Tensor) -> torch.Tensor:
    t = t.contiguous()
    return t.view(torch.uint8) if t.element_size() == 1 else t.view({2: torch.int16, 4: torch.int32}[t.element_size()])


def _selfcheck(key, fused_fn, stock_fn, *, last: bool = True) -> bool:  # noqa: ANN001
    """Once per key (site, width, ...): the fused producer against the stock pair on the first rows, bit for bit; a
    mismatch (or an exception) of the ``last`` candidate disables the site for the process."""
    ok = _state["checked"].get(key)
    if ok is not None:
        return ok
    try:
        fused, stock = fused_fn(), stock_fn()
        ok = len(fused) == len(stock) and all(
            f.shape == s.shape and f.dtype == s.dtype and torch.equal(_bits(f), _bits(s)) for f, s in zip(fused, stock))
    except Exception as exc:  # noqa: BLE001
        logger.warning("h3_tp2_amd fp8 quant: self-check %s raised %s: %s", key, type(exc).__name__, exc)
        ok = False
    _state["checked"][key] = ok
    if ok:
        _stats["selfcheck_pass"] += 1
    else:
        _stats["selfcheck_fail"] += 1
        if last:
            _state["disabled"].add(key[0])
        logger.warning("h3_tp2_amd fp8 quant: self-check %s not bit-identical to the stock pair; %s", key,
                       f"site {key[0]} disabled" if last else "trying the next mode")
    return ok


def _pick_mode(key, fused_for, stock_fn):  # noqa: ANN001,ANN202
    """The RMS-norm sites: mode 0 (bf16 row only in registers) if it passes the self-check, else mode 1 (the bf16 row
    stored too and compared as well); None when neither is bit-identical (the site is then disabled).  ``stock_fn``
    returns the stock outputs with the bf16 row last."""
    modes = _state["modes"]
    for m in modes:
        if _selfcheck(key + (m,), lambda: fused_for(m), lambda: stock_fn()[:None if m else -1], last=m == modes[-1]):
            return m
    return None


def _stock_quant(quant_obj, h: torch.Tensor):  # noqa: ANN001,ANN202
    """The layer's own per-token quant (the unwrapped ``QuantFP8.forward``), called as ``apply_weights`` calls it."""
    return _state["orig_quant"](quant_obj, h, None, None)


def _verify(p: Pending) -> None:
    """H3_TP2_AMD_QUANT_VERIFY=1: the stock pair on the full tensor against the stash (differences logged)."""
    h = p.materialize()
    q_ref, s_ref = _stock_quant(p.quant, h.view(-1, p.k))
    _stats["verify_calls"] += 1
    nq = int((_bits(p.q) != _bits(q_ref)).sum())
    ns = int((_bits(p.scale) != _bits(s_ref)).sum())
    if nq or ns:
        _stats["verify_mismatch"] += 1
        if _stats["verify_mismatch"] <= 20:
            logger.warning("h3_tp2_amd fp8 quant VERIFY: %s M=%d K=%d: %d fp8 bytes and %d scales differ",
                           p.site, h.numel() // p.k, p.k, nq, ns)


def make_quant_forward(orig):  # noqa: ANN001,ANN201
    """Wrap ``QuantFP8.forward``: the pending stash's (fp8, scale) for exactly its planned instance and placeholder;
    kernel 1 for the other dynamic per-token calls it takes (when enabled); ``orig`` for everything else."""
    def forward(self, x, *args, **kwargs):  # noqa: ANN001,ANN202
        scale = args[0] if args else kwargs.get("scale")
        scale_ub = args[1] if len(args) > 1 else kwargs.get("scale_ub")
        ctx = getattr(_tls, "ctx", None)
        p = ctx.pending if ctx is not None else None
        if p is not None:
            if scale is None and scale_ub is None and p.matches(self, x):
                ctx.pending = None
                if _state["verify"]:
                    _verify(p)
                _stats["consumed"] += 1
                return p.q, p.scale
            _materialize(ctx, "quant of another tensor")
        if (_state["kernel1"] and scale is None and scale_ub is None and dynamic_per_token(self)
                and kernel1_takes(x)):
            _stats["kernel1"] += 1
            return quant(x)
        _stats["stock_quant"] += 1
        return orig(self, x, *args, **kwargs)

    forward._h3_tp2_amd_quant = True
    forward.__wrapped__ = orig
    return forward


# ---- the block context and the fc2 producer site ----------------------------------------------------------------------

def _layer_post_hook(module, args, output):  # noqa: ANN001,ANN202
    """Safety net: a planned layer whose forward returned without its quant consuming the stash ran on the placeholder;
    make the placeholder real and run the layer again."""
    ctx = getattr(_tls, "ctx", None)
    p = ctx.pending if ctx is not None else None
    if p is None or p.layer is not module:
        return None
    _materialize(ctx, f"{p.site} layer returned without consuming")
    _stats["rerun"] += 1
    return module.forward(*args)


def _quant_of(layer):  # noqa: ANN001,ANN202
    """The layer's dynamic per-token QuantFP8 instance, or None."""
    kernel = getattr(getattr(layer, "quant_method", None), "fp8_linear", None)
    q = getattr(kernel, "quant_fp8", None)
    cls = _state["quant_cls"]
    if cls is None or not isinstance(q, cls) or not dynamic_per_token(q):
        return None
    if getattr(layer, "input_scale", None) is not None or getattr(layer, "input_scale_ub", None) is not None:
        return None
    return q


def block_plan(block, sites, lora_types=()) -> tuple[dict | None, str]:  # noqa: ANN001
    """{site: (layer, QuantFP8 instance)} for this block, or (None, reason)."""
    try:
        if torch.compiler.is_compiling():
            return None, "torch.compile tracing"
    except AttributeError:
        pass
    attn, mlp = getattr(block, "attn", None), getattr(block, "mlp", None)
    layers = {"qkv": getattr(attn, "qkv_proj", None), "out": getattr(attn, "out_proj", None),
              "fc1": getattr(mlp, "fc1", None), "fc2": getattr(mlp, "fc2", None)}
    plan: dict = {}
    for site in sites:
        if site in _state["disabled"]:
            continue
        layer = layers[site]
        if layer is None or (lora_types and isinstance(layer, lora_types)):
            return None, f"{site}: missing or LoRA-wrapped layer"
        if getattr(layer, "tp_size", 1) != 1:
            return None, f"{site}: tp_size != 1"
        q = _quant_of(layer)
        if q is None:
            return None, f"{site}: not a dynamic per-token FP8 linear"
        if site == "fc2" and _state["act_cls"] is not None and not isinstance(getattr(mlp, "act_fn", None),
                                                                              _state["act_cls"]):
            continue
        plan[site] = (layer, q)
        if not getattr(layer, "_h3_tp2_amd_quant_hook", False):
            layer.register_forward_hook(_layer_post_hook)
            layer._h3_tp2_amd_quant_hook = True
    return (plan or None), "no site left"


def make_block_forward(orig_forward, sites, lora_types=()):  # noqa: ANN001,ANN201
    @functools.wraps(orig_forward)
    def forward(self, *args, **kwargs):  # noqa: ANN001,ANN202
        plan, reason = block_plan(self, sites, lora_types)
        if plan is None:
            _warn_once("plan-" + reason, "block not fused (%s); stock path", reason)
            return orig_forward(self, *args, **kwargs)
        prev = getattr(_tls, "ctx", None)
        ctx = _Ctx(self, plan)
        _tls.ctx = ctx
        ok = False
        try:
            out = orig_forward(self, *args, **kwargs)
            ok = True
            return out
        finally:
            _tls.ctx = prev
            if ctx.pending is not None:
                if ok:
                    _materialize(ctx, "stash left at the end of the block")
                ctx.pending = None

    forward._h3_tp2_amd_quant = True
    return forward


def _take_site(site: str):  # noqa: ANN202
    """The running block's ctx when ``site`` is planned and enabled (a stash still pending is materialised first)."""
    ctx = getattr(_tls, "ctx", None)
    if ctx is None or site not in ctx.plan or site in _state["disabled"]:
        return None
    if ctx.pending is not None:
        _materialize(ctx, f"{site} producer while another stash was pending")
    return ctx


def _k_of(layer) -> int:  # noqa: ANN001
    """The layer's input width (weight [K, N] as vLLM stores it)."""
    w = getattr(layer, "weight", None)
    return int(w.shape[0]) if isinstance(w, torch.Tensor) and w.dim() == 2 else -1


def _rows_ok(x, k: int, *others) -> bool:  # noqa: ANN001
    """The reference's site precondition: x bf16 [M>0, k] contiguous; the other operands 2-D with unit column stride."""
    return (isinstance(x, torch.Tensor) and x.dim() == 2 and x.dtype == torch.bfloat16 and x.is_contiguous()
            and x.shape[0] > 0 and x.shape[1] == k
            and all(isinstance(o, torch.Tensor) and o.dim() == 2 and o.stride(1) == 1 for o in others))


def producer_takes(x, weight, tables, indices) -> bool:  # noqa: ANN001
    """Inputs the producer kernels take: bf16 on one CUDA device; x rows of width H (H % 8 == 0, H <= 8192) with
    16-byte aligned rows; weight a contiguous [H] vector; the [B, H] tables with 16-byte aligned rows; indices
    int32 / int64 [M]."""
    if not (isinstance(x, torch.Tensor) and x.is_cuda and x.dim() == 2 and x.dtype == torch.bfloat16):
        return False
    M, H = x.shape

    def rows16(t) -> bool:  # noqa: ANN001
        return (t.dim() == 2 and t.dtype == torch.bfloat16 and t.device == x.device and t.shape[1] == H
                and (H <= 1 or t.stride(1) == 1) and (t.shape[0] <= 1 or t.stride(0) % 8 == 0)
                and t.data_ptr() % 16 == 0)

    return (0 < H <= 8192 and H % 8 == 0 and rows16(x) and all(isinstance(t, torch.Tensor) and rows16(t) and
                                                                t.shape[0] > 0 for t in tables)
            and isinstance(weight, torch.Tensor) and weight.dtype == torch.bfloat16 and weight.device == x.device
            and weight.numel() == H and weight.is_contiguous() and weight.data_ptr() % 16 == 0
            and isinstance(indices, torch.Tensor) and indices.device == x.device and indices.dim() == 1
            and indices.shape[0] == M and indices.dtype in (torch.int32, torch.int64))


def make_own_rms(orig):  # noqa: ANN001,ANN201
    """``own_producers``: the stock ``rms_norm_indexed_scale_shift`` replaced by the producer kernel without the quant
    for the inputs it takes (``orig`` for the others)."""
    def rms_norm_indexed_scale_shift(x, weight, shift, scale, indices, eps):  # noqa: ANN001,ANN202
        if producer_takes(x, weight, (shift, scale), indices):
            _stats["own_producer"] += 1
            return ops.rms_norm_indexed_scale_shift(x, weight, shift, scale, indices, eps)
        return orig(x, weight, shift, scale, indices, eps)

    rms_norm_indexed_scale_shift._h3_tp2_amd_own = True
    rms_norm_indexed_scale_shift.__wrapped__ = orig
    return rms_norm_indexed_scale_shift


def make_own_gate_rms(orig):  # noqa: ANN001,ANN201
    """``own_producers``: the stock ``indexed_gate_rms_norm_scale_shift`` replaced by the producer kernel."""
    def indexed_gate_rms_norm_scale_shift(residual, gate, branch, weight, shift, scale, indices, eps):  # noqa: ANN001,ANN202
        if (producer_takes(residual, weight, (gate, shift, scale, branch), indices)
                and branch.shape == residual.shape):
            _stats["own_producer"] += 1
            return ops.indexed_gate_rms_norm_scale_shift(residual, gate, branch, weight, shift, scale, indices, eps)
        return orig(residual, gate, branch, weight, shift, scale, indices, eps)

    indexed_gate_rms_norm_scale_shift._h3_tp2_amd_own = True
    indexed_gate_rms_norm_scale_shift.__wrapped__ = orig
    return indexed_gate_rms_norm_scale_shift


def make_rms_wrapper(orig):  # noqa: ANN001,ANN201
    """``rms_norm_indexed_scale_shift`` (the block's norm1 + AdaLN before the QKV projection): the qkv site."""
    def rms_norm_indexed_scale_shift(x, weight, shift, scale, indices, eps):  # noqa: ANN001,ANN202
        ctx = _take_site("qkv")
        if ctx is not None:
            layer, qobj = ctx.plan["qkv"]
            blk = ctx.block
            if (weight is getattr(getattr(blk, "norm1", None), "weight", None)
                    and _rows_ok(x, _k_of(layer), shift, scale)
                    and producer_takes(x, weight, (shift, scale), indices)):
                r = min(_SELFCHECK_ROWS, x.shape[0])
                key = ("qkv", x.shape[1], shift.dtype, weight.dtype)

                def _fused_sub(mode):  # noqa: ANN001,ANN202
                    ph_r = torch.empty_like(x[:r]) if mode else None
                    q_r, s_r = rms_quant(x[:r], weight, shift, scale, indices[:r], eps, orig, ph_r)
                    return (q_r, s_r) + ((ph_r,) if mode else ())

                def _stock_sub():  # noqa: ANN202
                    h = orig(x[:r], weight, shift, scale, indices[:r], eps)
                    return (*_stock_quant(qobj, h), h)

                mode = _pick_mode(key, _fused_sub, _stock_sub)
                if mode is not None:
                    ph = torch.empty_like(x)
                    q, s = rms_quant(x, weight, shift, scale, indices, eps, orig, ph if mode else None)

                    def fill(t, _a=(x, weight, shift, scale, indices, eps)):  # noqa: ANN001,ANN202
                        t.copy_(orig(*_a))
                    ctx.pending = Pending("qkv", ph, x.shape[1], q, s, qobj, layer,
                                          (lambda t: None) if mode else fill)
                    _stats["fused_qkv"] += 1
                    return ph
        return orig(x, weight, shift, scale, indices, eps)

    rms_norm_indexed_scale_shift._h3_tp2_amd_quant = True
    rms_norm_indexed_scale_shift.__wrapped__ = orig
    return rms_norm_indexed_scale_shift


def make_gate_rms_wrapper(orig):  # noqa: ANN001,ANN201
    """``indexed_gate_rms_norm_scale_shift`` (the gated residual + norm2 + AdaLN before fc1): the fc1 site."""
    def indexed_gate_rms_norm_scale_shift(residual, gate, branch, weight, shift, scale, indices, eps):  # noqa: ANN001,ANN202
        ctx = _take_site("fc1")
        if ctx is not None:
            layer, qobj = ctx.plan["fc1"]
            blk = ctx.block
            if (weight is getattr(getattr(blk, "norm2", None), "weight", None)
                    and _rows_ok(residual, _k_of(layer), gate, branch, shift, scale)
                    and isinstance(branch, torch.Tensor) and branch.shape == residual.shape
                    and branch.dtype == residual.dtype
                    and producer_takes(residual, weight, (gate, branch, shift, scale), indices)):
                r = min(_SELFCHECK_ROWS, residual.shape[0])
                key = ("fc1", residual.shape[1], gate.dtype, weight.dtype)

                def _fused_sub(mode):  # noqa: ANN001,ANN202
                    ph_r = torch.empty_like(residual[:r]) if mode else None
                    out = gate_rms_quant(residual[:r], gate, branch[:r], weight, shift, scale, indices[:r], eps, orig,
                                         ph_r)
                    return out + ((ph_r,) if mode else ())

                def _stock_sub():  # noqa: ANN202
                    res, mod = orig(residual[:r], gate, branch[:r], weight, shift, scale, indices[:r], eps)
                    return (res, *_stock_quant(qobj, mod), mod)

                mode = _pick_mode(key, _fused_sub, _stock_sub)
                if mode is not None:
                    ph = torch.empty_like(residual)
                    res, q, s = gate_rms_quant(residual, gate, branch, weight, shift, scale, indices, eps, orig,
                                               ph if mode else None)

                    def fill(t, _a=(residual, gate, branch, weight, shift, scale, indices, eps)):  # noqa: ANN001,ANN202
                        t.copy_(orig(*_a)[1])
                    ctx.pending = Pending("fc1", ph, residual.shape[1], q, s, qobj, layer,
                                          (lambda t: None) if mode else fill)
                    _stats["fused_fc1"] += 1
                    return res, ph
        return orig(residual, gate, branch, weight, shift, scale, indices, eps)

    indexed_gate_rms_norm_scale_shift._h3_tp2_amd_quant = True
    indexed_gate_rms_norm_scale_shift.__wrapped__ = orig
    return indexed_gate_rms_norm_scale_shift


def make_act_forward(orig):  # noqa: ANN001,ANN201
    """``SiluAndMul.forward`` (the MLP's act_fn on fc1's bf16 output): the fc2 site."""
    def forward(self, x):  # noqa: ANN001,ANN202
        ctx = _take_site("fc2")
        if ctx is not None and self is getattr(getattr(ctx.block, "mlp", None), "act_fn", None):
            layer, qobj = ctx.plan["fc2"]
            if (isinstance(x, torch.Tensor) and x.is_cuda and x.dim() == 2 and x.dtype == torch.bfloat16
                    and x.is_contiguous() and x.shape[0] > 0 and x.shape[1] == 2 * _k_of(layer)
                    and x.shape[1] % 8 == 0):
                r = min(_SELFCHECK_ROWS, x.shape[0])
                if _selfcheck(("fc2", x.shape[1]), lambda: silu_mul_quant(x[:r]),
                              lambda: _stock_quant(qobj, orig(self, x[:r]))):
                    q, s = silu_mul_quant(x)
                    ph = torch.empty((x.shape[0], x.shape[1] // 2), dtype=x.dtype, device=x.device)

                    def fill(t, _x=x, _m=self):  # noqa: ANN001,ANN202
                        t.copy_(orig(_m, _x))
                    ctx.pending = Pending("fc2", ph, x.shape[1] // 2, q, s, qobj, layer, fill)
                    _stats["fused_fc2"] += 1
                    return ph
        return orig(self, x)

    forward._h3_tp2_amd_quant = True
    return forward


def parse_sites(value: str | None) -> tuple[str, ...]:
    """"1"/"all" = every site; a comma list of qkv,out,fc1,fc2; empty/"0"/"off" = none."""
    v = (value or "").strip().lower()
    if v in ("1", "all", "on", "true"):
        return SITES
    if not v or v in ("0", "off", "false"):
        return ()
    sel = {p.strip() for p in v.split(",")}
    return tuple(s for s in SITES if s in sel)


def install(sites=SITES, *, kernel1: bool = True, tr=None, quant_cls=None, act_cls=None,  # noqa: ANN001
            lora_types=None, own_producers: bool | None = None) -> list[str]:
    """Wrap ``QuantFP8.forward`` (kernel 1 for the dynamic per-token calls when ``kernel1``; stash consumption) and,
    for the wired producer sites among ``sites``, the block forward and the producers.  Returns the sites wired.
    ``own_producers`` (default: env H3_TP2_AMD_OWN_PRODUCERS=1) also replaces the stock RMS-norm producers by the
    producer kernels without the quant."""
    if isinstance(sites, str):
        sites = parse_sites(sites)
    if quant_cls is None:
        from vllm.model_executor.layers.quantization.input_quant_fp8 import QuantFP8 as quant_cls  # noqa: PLC0415
    _state["quant_cls"] = quant_cls
    _state["kernel1"] = bool(kernel1)
    _state["verify"] = os.environ.get("H3_TP2_AMD_QUANT_VERIFY", "0").strip() == "1"
    if not getattr(quant_cls.forward, "_h3_tp2_amd_quant", False):
        _state["orig_quant"] = quant_cls.forward
        quant_cls.forward = make_quant_forward(quant_cls.forward)
    for site in sites:
        if site not in WIRED_SITES:
            _warn_once("site-" + site, "site %s skipped: its producer kernel is not part of this library", site)
    sites = tuple(s for s in sites if s in WIRED_SITES)
    if not sites:
        return []
    if tr is None:
        from vllm_omni.diffusion.models.minimax_h3 import minimax_h3_transformer as tr  # noqa: PLC0415
    if "fc1" in sites and getattr(tr.indexed_gate_rms_norm_scale_shift, "_h3_tp2_amd_consumer", False):
        _warn_once("site-fc1-consumer", "site fc1 skipped: the consumer hook owns indexed_gate_rms_norm_scale_shift")
        sites = tuple(s for s in sites if s != "fc1")
        if not sites:
            return []
    if act_cls is None and "fc2" in sites:
        from vllm_omni.diffusion.layers.activation import SiluAndMul as act_cls  # noqa: PLC0415
    if lora_types is None:
        try:
            from vllm.lora.layers import BaseLayerWithLoRA  # noqa: PLC0415
            lora_types = (BaseLayerWithLoRA,)
        except ImportError:
            lora_types = ()
    _state["act_cls"] = act_cls if "fc2" in sites else None
    if "fc2" in sites and not getattr(act_cls.forward, "_h3_tp2_amd_quant", False):
        act_cls.forward = make_act_forward(act_cls.forward)
    if own_producers is None:
        own_producers = os.environ.get("H3_TP2_AMD_OWN_PRODUCERS", "0").strip() == "1"
    _state["own_producers"] = bool(own_producers)
    if own_producers:
        if not getattr(tr.rms_norm_indexed_scale_shift, "_h3_tp2_amd_own", False) and \
                not getattr(tr.rms_norm_indexed_scale_shift, "_h3_tp2_amd_quant", False):
            tr.rms_norm_indexed_scale_shift = make_own_rms(tr.rms_norm_indexed_scale_shift)
        if not getattr(tr.indexed_gate_rms_norm_scale_shift, "_h3_tp2_amd_own", False) and \
                not getattr(tr.indexed_gate_rms_norm_scale_shift, "_h3_tp2_amd_quant", False):
            tr.indexed_gate_rms_norm_scale_shift = make_own_gate_rms(tr.indexed_gate_rms_norm_scale_shift)
    if "qkv" in sites and not getattr(tr.rms_norm_indexed_scale_shift, "_h3_tp2_amd_quant", False):
        tr.rms_norm_indexed_scale_shift = make_rms_wrapper(tr.rms_norm_indexed_scale_shift)
    if "fc1" in sites and not getattr(tr.indexed_gate_rms_norm_scale_shift, "_h3_tp2_amd_quant", False):
        tr.indexed_gate_rms_norm_scale_shift = make_gate_rms_wrapper(tr.indexed_gate_rms_norm_scale_shift)
    mode = os.environ.get("H3_TP2_AMD_QUANT_MODE", "auto").strip().lower()
    _state["modes"] = {"0": (0,), "1": (1,)}.get(mode, (0, 1))
    block_cls = tr.MiniMaxH3DiTBlock
    if not getattr(block_cls.forward, "_h3_tp2_amd_quant", False):
        block_cls.forward = make_block_forward(block_cls.forward, sites, lora_types)
    _state["sites"] = sites
    return list(sites)


def stats() -> dict:
    return dict(_stats)
