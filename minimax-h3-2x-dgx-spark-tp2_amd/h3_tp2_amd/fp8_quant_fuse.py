"""Per-token dynamic FP8 activation quant on MI355X: the drop-in for ``QuantFP8.forward`` and the producer-fused
quant protocol.

The same protocol and names as the reference's h3_tp2/fp8_quant_fuse.py (``quant`` :318-327, ``rms_quant`` :330-346,
``gate_rms_quant`` :349-369, ``unpack_stock`` / ``unpack_quant`` :372-385, ``silu_mul_quant`` :392-402, ``Pending``
:432-450, ``make_quant_forward`` :553-576, ``block_plan`` :614-645, ``make_block_forward`` :648-670, ``parse_sites``
:836-844, ``install`` :925-1003), built here on a block scope object (``ProducerScope``), one generic engine for the
three producer sites (``_ProducerCall`` subclasses say how to recognise, run and check each producer) and the shared
verdict book of ``_sites``; compute on kernel 1, the producer kernels and the SwiGLU + quant kernel:

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

Producer bit identity.  The producer kernels sum the squares exactly (fp64, one rounding to fp32); a stock producer
that reduces in fp32 rounds some rows' sums differently (about 42 % of serving-like rows against torch's CPU fp32
sum), and on some of those its bf16 row differs by one ulp (1 % of the rows at H = 1024, 3 % at 3072, 4.5 % at 5376;
the fp8 bytes or scale on 0.07-0.18 %).  A self-check on the first rows cannot see every such row, so
``install`` wires the qkv / fc1 sites only when the stock producers are this library's own (``own_producers=True``, env
``H3_TP2_AMD_OWN_PRODUCERS=1``: the stock ``rms_norm_indexed_scale_shift`` / ``indexed_gate_rms_norm_scale_shift``
are replaced by the same kernels without the quant, so fused and stock agree by construction -- at the price of
those one-ulp differences against the upstream producers), or when the caller vouches for the stock producers'
reduction (``trust_selfcheck=True``).  Otherwise it logs that the two sites stay stock.  The fc2 site has no reduction
before its quant and is always eligible.  The out site (the Ulysses reverse exchange's unpack) exists only with
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

from . import _drift, _sites, ops

logger = logging.getLogger("h3_tp2_amd.fp8_quant_fuse")

E4M3 = torch.float8_e4m3fn
FP8_MAX = ops.FP8_MAX
MIN_SCALE = ops.MIN_SCALE
SITES = ("qkv", "out", "fc1", "fc2")
WIRED_SITES = ("qkv", "fc1", "fc2")
REDUCING_SITES = ("qkv", "fc1")          # producers with an RMS reduction before the quant
_SELFCHECK_ROWS = 64

_tls = threading.local()   # ctx: the ProducerScope of the DiT block whose forward is running in this thread
_state: dict[str, Any] = {"sites": (), "checked": {}, "disabled": set(), "orig_quant": None, "quant_cls": None,
                          "act_cls": None, "kernel1": False, "verify": False, "modes": (0, 1), "own_producers": False}
_stats: dict[str, int] = {"kernel1": 0, "stock_quant": 0, "fused_qkv": 0, "fused_fc1": 0, "fused_fc2": 0,
                          "consumed": 0, "materialize": 0, "rerun": 0, "selfcheck_pass": 0, "selfcheck_fail": 0,
                          "verify_calls": 0, "verify_mismatch": 0, "own_producer": 0}
_notes = _sites.Notes(logger, "h3_tp2_amd fp8 quant: ")
_warned = _notes.seen


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
    P, m, hl, d = recv.shape
    out = torch.empty((1, m, heads, d), dtype=recv.dtype, device=recv.device)
    out[0].view(m, P, hl, d).copy_(recv.permute(1, 0, 2, 3))
    return out


def unpack_quant(recv: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """The unpack + the per-token quant of the [M, P*hl*d] out-projection input, read straight from the receive buffer
    [P, M, hl, d] (kernel 1 on P segments): (fp8 [M, P*hl*d], scale [M, 1])."""
    return ops.quant_from_recv(recv)


def silu_mul_quant(x: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """silu(x[:, :d]) * x[:, d:] on bf16 [M, 2d] (each product rounded to bf16) + the per-token quant of the [M, d]
    result: (fp8 [M, d], fp32 scale [M, 1])."""
    return ops.silu_mul_quant(x)


# ---- what the quant drop-in and the producer kernels take -------------------------------------------------------------

def dynamic_per_token(quant_obj) -> bool:  # noqa: ANN001
    """True for a ``QuantFP8`` instance that computes a dynamic per-token scale (the only form kernel 1 replaces):
    not static, per token, no group quant, no token padding (the attribute checks of fp8_quant_fuse.py:596-600)."""
    flags = (getattr(quant_obj, "static", True), getattr(quant_obj, "use_per_token_if_dynamic", False),
             getattr(quant_obj, "is_group_quant", True), getattr(quant_obj, "num_token_padding", 0))
    return flags[:3] == (False, True, False) and flags[3] is None


def _rows16(t: torch.Tensor, like: torch.Tensor, width: int) -> bool:
    """bf16 rows of ``width`` on ``like``'s device, unit column stride, row stride a multiple of 8, 16-byte aligned."""
    return (isinstance(t, torch.Tensor) and t.dim() == 2 and t.dtype == torch.bfloat16 and t.device == like.device
            and t.shape[1] == width and (width <= 1 or t.stride(1) == 1) and (t.shape[0] <= 1 or t.stride(0) % 8 == 0)
            and t.data_ptr() % 16 == 0)


def kernel1_takes(x) -> bool:  # noqa: ANN001
    """Inputs kernel 1 takes: a bf16 CUDA tensor of 2 dims with contiguous rows, K % 8 == 0, 16-byte aligned rows."""
    return isinstance(x, torch.Tensor) and x.is_cuda and x.dim() == 2 and x.shape[1] % 8 == 0 and \
        _rows16(x, x, x.shape[1])


def producer_takes(x, weight, tables, indices) -> bool:  # noqa: ANN001
    """Inputs the producer kernels take: bf16 on one CUDA device; x rows of width H (H % 8 == 0, H <= 8192) with
    16-byte aligned rows; weight a contiguous [H] vector; the [B, H] tables with 16-byte aligned rows; indices
    int32 / int64 [M]."""
    if not (isinstance(x, torch.Tensor) and x.is_cuda and x.dim() == 2 and x.dtype == torch.bfloat16):
        return False
    M, H = x.shape
    weight_ok = (isinstance(weight, torch.Tensor) and weight.dtype == torch.bfloat16 and weight.device == x.device
                 and weight.numel() == H and weight.is_contiguous() and weight.data_ptr() % 16 == 0)
    index_ok = (isinstance(indices, torch.Tensor) and indices.device == x.device and indices.dim() == 1
                and indices.shape[0] == M and indices.dtype in (torch.int32, torch.int64))
    return (0 < H <= 8192 and H % 8 == 0 and _rows16(x, x, H) and weight_ok and index_ok
            and all(_rows16(t, x, H) and t.shape[0] > 0 for t in tables))


# ---- the stash and the block scope ------------------------------------------------------------------------------------

class Pending:
    """A producer's (fp8, scale) waiting for the quant of ``layer``; ``ph`` is the bf16 placeholder the model holds and
    ``k`` the GEMM input width (the quant sees ``ph`` as a contiguous [numel / k, k] view).  ``fill`` writes the stock
    producer's bf16 output into a placeholder (``materialize``)."""
    __slots__ = ("site", "ph", "k", "q", "scale", "quant", "layer", "fill", "_view")

    def __init__(self, site: str, ph: torch.Tensor, k: int, q: torch.Tensor, scale: torch.Tensor, quant_obj,  # noqa: ANN001
                 layer, fill: Callable[[torch.Tensor], None]):
        self.site, self.ph, self.k, self.q, self.scale = site, ph, k, q, scale
        self.quant, self.layer, self.fill = quant_obj, layer, fill
        # the one view of the placeholder its quant may be called on: (address, dtype, device, shape, strides)
        self._view = ((ph.data_ptr(), ph.dtype, ph.device, (ph.numel() // k, k), (k, 1))
                      if ph.is_contiguous() else None)

    def matches(self, quant_obj, x) -> bool:  # noqa: ANN001
        if quant_obj is not self.quant or self._view is None or not isinstance(x, torch.Tensor) or x.dim() != 2:
            return False
        return (x.data_ptr(), x.dtype, x.device, tuple(x.shape), x.stride()) == self._view

    def materialize(self) -> torch.Tensor:
        self.fill(self.ph)
        return self.ph


class ProducerScope:
    """One DiT block's forward: the planned sites (``plan``: site -> (layer, its QuantFP8 instance)) and at most one
    stash waiting for its quant (``pending``)."""
    __slots__ = ("block", "plan", "pending")

    def __init__(self, block, plan: dict):  # noqa: ANN001
        self.block, self.plan = block, plan
        self.pending: Pending | None = None

    def release(self, reason: str) -> None:
        """Materialise the waiting stash, if any: its layer's quant will then run the stock way on the bf16 row."""
        p, self.pending = self.pending, None
        if p is None:
            return
        p.materialize()
        _stats["materialize"] += 1
        _notes.once("mat-" + reason, "%s: the %s stash is replaced by the stock producer's bf16 row", reason, p.site)

    def open_for(self, site: str) -> bool:
        """True when ``site`` is planned and enabled; a stash still waiting is materialised first."""
        if site not in self.plan or site in _state["disabled"]:
            return False
        self.release(f"the {site} producer ran while an earlier stash still waited")
        return True

    def close(self) -> None:
        """The block returned: a stash nobody consumed gets its bf16 row for whoever still holds the placeholder."""
        self.release("the block returned with its stash unconsumed")

    def drop(self) -> None:
        """The block raised: nothing will read the placeholder."""
        self.pending = None


_Ctx = ProducerScope          # the name the protocol tests address


def _scope() -> ProducerScope | None:
    return getattr(_tls, "ctx", None)


# ---- the QuantFP8 drop-in ---------------------------------------------------------------------------------------------

def _stock_quant(quant_obj, h: torch.Tensor):  # noqa: ANN001,ANN202
    """The per-token quant the layer would run without this module (the original ``QuantFP8.forward``), with the
    arguments ``apply_weights`` passes."""
    return _state["orig_quant"](quant_obj, h, None, None)


def _verify(p: Pending) -> None:
    """H3_TP2_AMD_QUANT_VERIFY=1: the stock pair on the full tensor against the stash (differences logged)."""
    h = p.materialize()
    q_ref, s_ref = _stock_quant(p.quant, h.view(-1, p.k))
    _stats["verify_calls"] += 1
    diff = [int(torch.count_nonzero(_sites._raw(a) != _sites._raw(b))) for a, b in ((p.q, q_ref), (p.scale, s_ref))]
    if any(diff):
        _stats["verify_mismatch"] += 1
        if _stats["verify_mismatch"] <= 20:
            logger.warning("h3_tp2_amd fp8 quant VERIFY: %s M=%d K=%d: %d fp8 bytes and %d scales differ",
                           p.site, h.numel() // p.k, p.k, *diff)


def make_quant_forward(orig):  # noqa: ANN001,ANN201
    """Wrap ``QuantFP8.forward``: the waiting stash's (fp8, scale) for exactly its planned instance and placeholder;
    kernel 1 for the other dynamic per-token calls it takes (when enabled); ``orig`` for everything else."""
    def forward(self, x, *args, **kwargs):  # noqa: ANN001,ANN202
        scale = args[0] if args else kwargs.get("scale")
        scale_ub = args[1] if len(args) > 1 else kwargs.get("scale_ub")
        dynamic = scale is None and scale_ub is None
        scope = _scope()
        waiting = scope.pending if scope is not None else None
        if waiting is not None:
            if dynamic and waiting.matches(self, x):
                scope.pending = None
                if _state["verify"]:
                    _verify(waiting)
                _stats["consumed"] += 1
                return waiting.q, waiting.scale
            scope.release("a quant of some other tensor came first")
        if dynamic and _state["kernel1"] and dynamic_per_token(self) and kernel1_takes(x):
            _stats["kernel1"] += 1
            return quant(x)
        _stats["stock_quant"] += 1
        return orig(self, x, *args, **kwargs)

    forward._h3_tp2_amd_quant = True
    forward.__wrapped__ = orig
    return forward


# ---- planning a block -------------------------------------------------------------------------------------------------

def _layer_post_hook(module, args, output):  # noqa: ANN001,ANN202
    """Safety net: a planned layer whose forward returned without its quant consuming the stash ran on the placeholder;
    make the placeholder real and run the layer again."""
    scope = _scope()
    waiting = scope.pending if scope is not None else None
    if waiting is None or waiting.layer is not module:
        return None
    scope.release(f"the {waiting.site} layer returned without taking its stash")
    _stats["rerun"] += 1
    return module.forward(*args)


def _quant_of(layer):  # noqa: ANN001,ANN202
    """The layer's dynamic per-token QuantFP8 instance, or None (static scales, scale bounds, other classes)."""
    q = getattr(getattr(getattr(layer, "quant_method", None), "fp8_linear", None), "quant_fp8", None)
    cls = _state["quant_cls"]
    has_static = any(getattr(layer, name, None) is not None for name in ("input_scale", "input_scale_ub"))
    return q if cls is not None and isinstance(q, cls) and dynamic_per_token(q) and not has_static else None


def _producer_refusal(site: str, layer, lora_types) -> str | None:  # noqa: ANN001
    """Why ``site``'s layer cannot take its input from a fused producer (None: it can): the shared layer rules, and
    its input quant must be a dynamic per-token QuantFP8 (the stash replaces exactly that call)."""
    why = _sites.layer_refusal(site, layer, lora_types)
    if why is None and _quant_of(layer) is None:
        why = f"{site}: its input is not quantised dynamically per token"
    return why


def _site_applies(block, site: str) -> bool:
    """The fc2 site wraps SiluAndMul: a block whose MLP activation is something else has no fc2 producer to fuse."""
    act_cls = _state["act_cls"]
    if site != "fc2" or act_cls is None:
        return True
    return isinstance(getattr(getattr(block, "mlp", None), "act_fn", None), act_cls)


def _watch(layer) -> None:  # noqa: ANN001
    """Hang the safety net (``_layer_post_hook``) on a planned layer, once."""
    if not getattr(layer, "_h3_tp2_amd_quant_hook", False):
        layer.register_forward_hook(_layer_post_hook)
        layer._h3_tp2_amd_quant_hook = True


def block_plan(block, sites, lora_types=()) -> tuple[dict | None, str]:  # noqa: ANN001
    """The producer sites of this block, as {site: (layer, its QuantFP8 instance)}, or (None, why not).  Every site
    still enabled must qualify, or the block runs stock."""
    if _sites.tracing():
        return None, "inside a torch.compile trace"
    layers = {site: _sites.site_layer(block, site) for site in sites if site not in _state["disabled"]}
    refusals = [why for why in (_producer_refusal(site, layer, lora_types) for site, layer in layers.items()) if why]
    if refusals:
        return None, refusals[0]
    plan = {site: (layer, _quant_of(layer)) for site, layer in layers.items() if _site_applies(block, site)}
    for layer, _ in plan.values():
        _watch(layer)
    return (plan or None), "every site is disabled or inapplicable"


def make_block_forward(orig_forward, sites, lora_types=()):  # noqa: ANN001,ANN201
    """Run a DiT block's forward inside a ProducerScope (``_sites.block_scope``: thread-local, nested blocks restore the
    outer scope, a stash left waiting at the end is computed the stock way)."""
    @functools.wraps(orig_forward)
    def forward(self, *args, **kwargs):  # noqa: ANN001,ANN202
        plan, why = block_plan(self, sites, lora_types)
        if plan is None:
            _notes.once("plan-" + why, "%s: this block's producers run stock", why)
            return orig_forward(self, *args, **kwargs)
        with _sites.block_scope(_tls, ProducerScope(self, plan)):
            return orig_forward(self, *args, **kwargs)

    forward._h3_tp2_amd_quant = True
    return forward


# ---- the producer sites -----------------------------------------------------------------------------------------------

def _k_of(layer) -> int:  # noqa: ANN001
    """K, the width of the layer's input (vLLM keeps the weight as [K, N])."""
    w = getattr(layer, "weight", None)
    return int(w.shape[0]) if isinstance(w, torch.Tensor) and w.dim() == 2 else -1


def _rows_ok(x, k: int, *others) -> bool:  # noqa: ANN001
    """The reference's site precondition: x bf16 [M>0, k] contiguous; the other operands 2-D with unit column stride."""
    return (isinstance(x, torch.Tensor) and x.dim() == 2 and x.dtype == torch.bfloat16 and x.is_contiguous()
            and x.shape[0] > 0 and x.shape[1] == k
            and all(isinstance(o, torch.Tensor) and o.dim() == 2 and o.stride(1) == 1 for o in others))


class _ProducerCall:
    """One call of a producer at a site: ``rows`` is the bf16 input whose rows the output follows; ``accepts(scope,
    layer)`` says whether the fused form may take it; ``fused(r, ph)`` runs the fused kernel on the first r rows (all
    rows: r None) and returns its outputs with (fp8, scale) last; ``stock(orig, r)`` runs the stock producer and
    returns its outputs with the bf16 row last; ``reply(extra, ph)`` is what the caller receives from the fused form."""
    site = ""
    modes: tuple | None = None                  # None: the configured modes (0: bf16 row in registers, 1: also stored)

    def key(self) -> tuple:
        raise NotImplementedError

    def accepts(self, scope: ProducerScope, layer) -> bool:  # noqa: ANN001
        raise NotImplementedError

    def fused(self, r, ph):  # noqa: ANN001,ANN201
        raise NotImplementedError

    def stock(self, orig, r):  # noqa: ANN001,ANN201
        raise NotImplementedError

    def reply(self, extra: tuple, ph: torch.Tensor):  # noqa: ANN201
        raise NotImplementedError

    def placeholder(self) -> torch.Tensor:
        return torch.empty_like(self.rows)


class _RmsCall(_ProducerCall):
    """``rms_norm_indexed_scale_shift(x, weight, shift, scale, indices, eps)``: the block's norm1 + AdaLN, the QKV
    projection's input (the qkv site)."""
    site = "qkv"

    def __init__(self, x, weight, shift, scale, indices, eps):  # noqa: ANN001
        self.args = (x, weight, shift, scale, indices, eps)
        self.rows = x

    def key(self) -> tuple:
        x, weight, shift = self.args[:3]
        return ("qkv", x.shape[1], shift.dtype, weight.dtype)

    def accepts(self, scope, layer) -> bool:  # noqa: ANN001
        x, weight, shift, scale, indices, _ = self.args
        norm1 = getattr(getattr(scope.block, "norm1", None), "weight", None)
        return (weight is norm1 and _rows_ok(x, _k_of(layer), shift, scale)
                and producer_takes(x, weight, (shift, scale), indices))

    def _sliced(self, r):  # noqa: ANN001,ANN202
        x, weight, shift, scale, indices, eps = self.args
        return (x, weight, shift, scale, indices, eps) if r is None else (x[:r], weight, shift, scale, indices[:r], eps)

    def fused(self, r, ph):  # noqa: ANN001,ANN201
        return rms_quant(*self._sliced(r), self._orig, ph)

    def stock(self, orig, r):  # noqa: ANN001,ANN201
        return (orig(*self._sliced(r)),)

    def reply(self, extra, ph):  # noqa: ANN001,ANN201
        return ph


class _GateRmsCall(_ProducerCall):
    """``indexed_gate_rms_norm_scale_shift(residual, gate, branch, weight, shift, scale, indices, eps)``: the gated
    residual + norm2 + AdaLN, fc1's input (the fc1 site); its residual_out goes back to the caller in both forms."""
    site = "fc1"

    def __init__(self, residual, gate, branch, weight, shift, scale, indices, eps):  # noqa: ANN001
        self.args = (residual, gate, branch, weight, shift, scale, indices, eps)
        self.rows = residual

    def key(self) -> tuple:
        residual, gate, _, weight = self.args[:4]
        return ("fc1", residual.shape[1], gate.dtype, weight.dtype)

    def accepts(self, scope, layer) -> bool:  # noqa: ANN001
        residual, gate, branch, weight, shift, scale, indices, _ = self.args
        norm2 = getattr(getattr(scope.block, "norm2", None), "weight", None)
        return (weight is norm2 and _rows_ok(residual, _k_of(layer), gate, branch, shift, scale)
                and isinstance(branch, torch.Tensor) and branch.shape == residual.shape
                and branch.dtype == residual.dtype
                and producer_takes(residual, weight, (gate, branch, shift, scale), indices))

    def _sliced(self, r):  # noqa: ANN001,ANN202
        residual, gate, branch, weight, shift, scale, indices, eps = self.args
        if r is None:
            return self.args
        return (residual[:r], gate, branch[:r], weight, shift, scale, indices[:r], eps)

    def fused(self, r, ph):  # noqa: ANN001,ANN201
        return gate_rms_quant(*self._sliced(r), self._orig, ph)

    def stock(self, orig, r):  # noqa: ANN001,ANN201
        return tuple(orig(*self._sliced(r)))

    def reply(self, extra, ph):  # noqa: ANN001,ANN201
        return extra[0], ph


class _SiluMulCall(_ProducerCall):
    """``SiluAndMul.forward(self, x)`` on fc1's bf16 output, fc2's input (the fc2 site): one form only (the bf16 row is
    never stored; materialising re-runs the stock activation)."""
    site = "fc2"
    modes = (0,)

    def __init__(self, act, x):  # noqa: ANN001
        self.act, self.x = act, x
        self.rows = x

    def key(self) -> tuple:
        return ("fc2", self.x.shape[1])

    def accepts(self, scope, layer) -> bool:  # noqa: ANN001
        x = self.x
        return (self.act is getattr(getattr(scope.block, "mlp", None), "act_fn", None) and isinstance(x, torch.Tensor)
                and x.is_cuda and x.dim() == 2 and x.dtype == torch.bfloat16 and x.is_contiguous() and x.shape[0] > 0
                and x.shape[1] == 2 * _k_of(layer) and x.shape[1] % 8 == 0)

    def fused(self, r, ph):  # noqa: ANN001,ANN201
        return silu_mul_quant(self.x if r is None else self.x[:r])

    def stock(self, orig, r):  # noqa: ANN001,ANN201
        return (orig(self.act, self.x if r is None else self.x[:r]),)

    def reply(self, extra, ph):  # noqa: ANN001,ANN201
        return ph

    def placeholder(self) -> torch.Tensor:
        x = self.x
        return torch.empty((x.shape[0], x.shape[1] // 2), dtype=x.dtype, device=x.device)


def _choose_mode(call: _ProducerCall, orig, qobj) -> int | None:  # noqa: ANN001
    """The first mode whose fused outputs equal the stock producer + the layer's own quant bit for bit on the first rows
    (checked once per key and mode); None when no mode does (the site is then disabled)."""
    r = min(_SELFCHECK_ROWS, call.rows.shape[0])
    modes = call.modes if call.modes is not None else _state["modes"]
    for i, mode in enumerate(modes):
        def fused(mode=mode):  # noqa: ANN001,ANN202
            ph_r = torch.empty_like(call.rows[:r]) if mode else None
            out = tuple(call.fused(r, ph_r))
            return out + (ph_r,) if mode else out

        def stock(mode=mode):  # noqa: ANN001,ANN202
            *extra, row = call.stock(orig, r)
            q, s = _stock_quant(qobj, row)
            return (*extra, q, s, row) if mode else (*extra, q, s)

        if _sites.checked(_state, _stats, _notes, call.key() + (mode,), fused, stock,
                          disable_site=i == len(modes) - 1):
            return mode
    return None


def _engage(call: _ProducerCall, orig):  # noqa: ANN001,ANN202
    """The fused form of one producer call at its site, or None (the caller runs the stock producer)."""
    scope = _scope()
    if scope is None or not scope.open_for(call.site):
        return None
    layer, qobj = scope.plan[call.site]
    call._orig = orig
    if not call.accepts(scope, layer):
        return None
    mode = _choose_mode(call, orig, qobj)
    if mode is None:
        return None
    ph = call.placeholder()
    *extra, q, s = call.fused(None, ph if mode else None)
    if mode:
        fill = _no_fill                                # the kernel already stored the bf16 row
    else:
        def fill(t, _call=call, _orig=orig):  # noqa: ANN001,ANN202
            t.copy_(_call.stock(_orig, None)[-1])
    scope.pending = Pending(call.site, ph, ph.shape[1], q, s, qobj, layer, fill)
    _stats["fused_" + call.site] += 1
    return call.reply(tuple(extra), ph)


def _no_fill(t: torch.Tensor) -> None:
    del t


def make_rms_wrapper(orig):  # noqa: ANN001,ANN201
    """``rms_norm_indexed_scale_shift`` (the block's norm1 + AdaLN before the QKV projection): the qkv site."""
    def rms_norm_indexed_scale_shift(x, weight, shift, scale, indices, eps):  # noqa: ANN001,ANN202
        out = _engage(_RmsCall(x, weight, shift, scale, indices, eps), orig)
        return out if out is not None else orig(x, weight, shift, scale, indices, eps)

    rms_norm_indexed_scale_shift._h3_tp2_amd_quant = True
    rms_norm_indexed_scale_shift.__wrapped__ = orig
    return rms_norm_indexed_scale_shift


def make_gate_rms_wrapper(orig):  # noqa: ANN001,ANN201
    """``indexed_gate_rms_norm_scale_shift`` (the gated residual + norm2 + AdaLN before fc1): the fc1 site."""
    def indexed_gate_rms_norm_scale_shift(residual, gate, branch, weight, shift, scale, indices, eps):  # noqa: ANN001,ANN202
        args = (residual, gate, branch, weight, shift, scale, indices, eps)
        out = _engage(_GateRmsCall(*args), orig)
        return out if out is not None else orig(*args)

    indexed_gate_rms_norm_scale_shift._h3_tp2_amd_quant = True
    indexed_gate_rms_norm_scale_shift.__wrapped__ = orig
    return indexed_gate_rms_norm_scale_shift


def make_act_forward(orig):  # noqa: ANN001,ANN201
    """The fc2 site's producer: the MLP's ``SiluAndMul.forward`` (act_fn, applied to fc1's bf16 output)."""
    def forward(self, x):  # noqa: ANN001,ANN202
        out = _engage(_SiluMulCall(self, x), orig)
        return out if out is not None else orig(self, x)

    forward._h3_tp2_amd_quant = True
    return forward


# ---- own producers: the stock RMS-norm producers replaced by the kernels without the quant -----------------------------

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


# ---- install ----------------------------------------------------------------------------------------------------------

def parse_sites(value: str | None) -> tuple[str, ...]:
    """"1"/"all" = every site; a comma list of qkv,out,fc1,fc2; empty/"0"/"off" = none."""
    return _sites.parse_site_list(value, SITES)


def _replace(module, name: str, factory, *marks: str) -> None:  # noqa: ANN001
    """module.name = factory(module.name), unless the current function already carries one of ``marks``."""
    current = getattr(module, name)
    if not any(getattr(current, m, False) for m in marks):
        setattr(module, name, factory(current))


def _lora_base_types() -> tuple:
    try:
        from vllm.lora.layers import BaseLayerWithLoRA  # noqa: PLC0415
    except ImportError:
        return ()
    return (BaseLayerWithLoRA,)


def _env_flag(name: str) -> bool:
    return os.environ.get(name, "0").strip() == "1"


def install(sites=SITES, *, kernel1: bool = True, tr=None, quant_cls=None, act_cls=None,  # noqa: ANN001
            lora_types=None, own_producers: bool | None = None, trust_selfcheck: bool = False,
            check_source: bool = True, reviewed: dict | None = None, modules: dict | None = None) -> list[str]:
    """Wrap ``QuantFP8.forward`` (kernel 1 for the dynamic per-token calls when ``kernel1``; stash consumption) and,
    for the wired producer sites among ``sites``, the block forward and the producers.  Returns the sites wired.

    ``own_producers`` (default: env H3_TP2_AMD_OWN_PRODUCERS=1) replaces the stock RMS-norm producers by the producer
    kernels without the quant, which makes the qkv / fc1 sites bit-identical to their stock by construction.  Without
    it those two sites are wired only with ``trust_selfcheck`` (the caller vouches that the stock producers reduce like
    the kernels); otherwise they stay stock, with a warning (see the module docstring).  With ``check_source`` a site
    is wired only when the upstream functions between its producer and its quant fingerprint to the reviewed sources
    (``_drift``; ``reviewed`` / ``modules`` override the table and the upstream modules)."""
    if isinstance(sites, str):
        sites = parse_sites(sites)
    if quant_cls is None:
        from vllm.model_executor.layers.quantization.input_quant_fp8 import QuantFP8 as quant_cls  # noqa: PLC0415
    _state.update(quant_cls=quant_cls, kernel1=bool(kernel1), verify=_env_flag("H3_TP2_AMD_QUANT_VERIFY"))
    if not getattr(quant_cls.forward, "_h3_tp2_amd_quant", False):
        _state["orig_quant"] = quant_cls.forward
        quant_cls.forward = make_quant_forward(quant_cls.forward)
    for site in sites:
        if site not in WIRED_SITES:
            _notes.once("site-" + site, "site %s skipped: its producer kernel is not part of this library", site)
    chosen = [s for s in sites if s in WIRED_SITES]
    if own_producers is None:
        own_producers = _env_flag("H3_TP2_AMD_OWN_PRODUCERS")
    _state["own_producers"] = bool(own_producers)
    if not own_producers and not trust_selfcheck:
        for site in (s for s in chosen if s in REDUCING_SITES):
            _notes.once("stock-" + site, "site %s stays stock: the fused producer sums the squares in fp64 and can "
                        "differ by one bf16 ulp from a stock fp32 reduction on rows the self-check does not sample; "
                        "own_producers=True (H3_TP2_AMD_OWN_PRODUCERS=1) uses the kernels for both", site)
        chosen = [s for s in chosen if s not in REDUCING_SITES]
    if not chosen:
        return []
    if tr is None:
        from vllm_omni.diffusion.models.minimax_h3 import minimax_h3_transformer as tr  # noqa: PLC0415
    if check_source:
        chosen = list(_drift.keep_sites("producers", chosen, tr, _notes, reviewed, modules))
        if not chosen:
            return []
    if "fc1" in chosen and getattr(tr.indexed_gate_rms_norm_scale_shift, "_h3_tp2_amd_consumer", False):
        _notes.once("site-fc1-consumer", "site fc1 skipped: the consumer hook owns indexed_gate_rms_norm_scale_shift")
        chosen.remove("fc1")
        if not chosen:
            return []
    if act_cls is None and "fc2" in chosen:
        from vllm_omni.diffusion.layers.activation import SiluAndMul as act_cls  # noqa: PLC0415
    _state["act_cls"] = act_cls if "fc2" in chosen else None
    if "fc2" in chosen and not getattr(act_cls.forward, "_h3_tp2_amd_quant", False):
        act_cls.forward = make_act_forward(act_cls.forward)
    if own_producers:
        _replace(tr, "rms_norm_indexed_scale_shift", make_own_rms, "_h3_tp2_amd_own", "_h3_tp2_amd_quant")
        _replace(tr, "indexed_gate_rms_norm_scale_shift", make_own_gate_rms, "_h3_tp2_amd_own", "_h3_tp2_amd_quant")
    if "qkv" in chosen:
        _replace(tr, "rms_norm_indexed_scale_shift", make_rms_wrapper, "_h3_tp2_amd_quant")
    if "fc1" in chosen:
        _replace(tr, "indexed_gate_rms_norm_scale_shift", make_gate_rms_wrapper, "_h3_tp2_amd_quant")
    _state["modes"] = {"0": (0,), "1": (1,)}.get(os.environ.get("H3_TP2_AMD_QUANT_MODE", "auto").strip().lower(),
                                                  (0, 1))
    block_cls = tr.MiniMaxH3DiTBlock
    if not getattr(block_cls.forward, "_h3_tp2_amd_quant", False):
        block_cls.forward = make_block_forward(block_cls.forward, tuple(chosen),
                                               _lora_base_types() if lora_types is None else lora_types)
    _state["sites"] = tuple(chosen)
    return list(chosen)


def stats() -> dict:
    return dict(_stats)
