"""The GEMM-output stash protocol of the DiT block on MI355X (the consumer side of the dispatcher's stash hooks).

The same protocol and names as the reference's h3_tp2/fp8_consumers.py (``Stash`` :388-399, ``scale_pass_into``
:373-380, ``stash_hook`` :531-546, the consumer wrappers :651-747, ``block_plan`` :758-784, ``make_block_forward``
:787-808, ``parse_sites`` :811-819, ``install`` :859-916), built here on a block scope object (``ConsumerScope``), one
self-checked fused-consumer class for the three sites and the shared verdict book of ``_sites``; compute on the HIP
kernels:

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

from . import _drift, _sites, fp8_gemm

logger = logging.getLogger("h3_tp2_amd.fp8_consumers")

SITES = ("qkv", "out", "fc2")
CONSUMERS = {"qkv": "fused_qk_norm_rope", "out": "indexed_gate_rms_norm_scale_shift", "fc2": "indexed_gate"}
HEAD_DIM = 128
ROTARY_DIM = 96
_SELFCHECK_ROWS = 64

_tls = threading.local()   # ctx: the ConsumerScope of the DiT block whose forward is running in this thread
# checked / disabled: the verdict book of the self-checks; fused: site -> registered fused consumer
_state: dict[str, Any] = {"sites": (), "disabled": set(), "fused": {}, "checked": {}}
_stats = {"stash": 0, "fused": 0, "materialize": 0, "stock": 0, "fused_qkv": 0, "fused_out": 0, "fused_fc2": 0,
          "selfcheck_pass": 0, "selfcheck_fail": 0}
_notes = _sites.Notes(logger, "h3_tp2_amd fp8 consumers: ")


def scale_pass_into(x32: torch.Tensor, sa: torch.Tensor, sb: torch.Tensor, bias: torch.Tensor | None,
                    y: torch.Tensor) -> torch.Tensor:
    """The ordinary scale pass into ``y`` (the stock output of the two-pass GEMM), on the device."""
    return fp8_gemm._launch(x32, sa, sb, bias, y, x32.shape[1])


class Stash:
    """What the stash hook keeps instead of running the scale pass: the GEMM's raw fp32 product, its per-token and
    per-channel scales and bias, and ``ph``, the uninitialised bf16 tensor handed to the model in its place."""
    __slots__ = ("x32", "sa", "sb", "bias", "ph")

    def __init__(self, x32: torch.Tensor, sa: torch.Tensor, sb: torch.Tensor, bias: torch.Tensor | None,
                 ph: torch.Tensor):
        self.x32, self.sa, self.sb, self.bias, self.ph = x32, sa, sb, bias, ph

    def materialize(self) -> torch.Tensor:
        """Write the stock output (the scale pass) into the placeholder and return it."""
        return scale_pass_into(self.x32, self.sa, self.sb, self.bias, self.ph)

    def rows(self, r: int) -> "Stash":
        """The first r rows as a stash of their own (its own placeholder): the self-checks' sample."""
        return Stash(self.x32[:r], self.sa[:r], self.sb, self.bias, torch.empty_like(self.ph[:r]))


class ConsumerScope:
    """One DiT block's forward: the weights whose GEMMs may be stashed (``want``: weight key -> site, each taken at most
    once) and the stashes waiting for their consumers (``pending``: site -> Stash)."""
    __slots__ = ("want", "pending")

    def __init__(self, want: dict):
        self.want = want
        self.pending: dict[str, Stash] = {}

    def flush(self, reason: str) -> None:
        """Materialise every waiting stash: their consumers will run the stock way."""
        for site, st in list(self.pending.items()):
            st.materialize()
            _stats["materialize"] += 1
            _notes.once("mat-" + reason, "%s: the %s output was computed after all (its consumer runs stock)", reason,
                        site)
        self.pending.clear()

    def claim(self, site: str) -> Stash | None:
        """The stash waiting for ``site``'s consumer (it stays registered until ``settle``); a consumer that finds only
        other sites' stashes makes them real first."""
        if not self.pending:
            return None
        st = self.pending.get(site)
        if st is None:
            self.flush(f"the {site} consumer found a stash of another site")
        return st

    def settle(self, site: str) -> None:
        self.pending.pop(site, None)

    def close(self) -> None:
        """The block returned: a stash nobody consumed is computed for whoever still holds its placeholder."""
        self.flush("the block returned with its stash unconsumed")

    def drop(self) -> None:
        """The block raised: nothing will read the placeholders."""
        self.pending.clear()


_Ctx = ConsumerScope          # the name the protocol tests address


def _scope() -> ConsumerScope | None:
    return getattr(_tls, "ctx", None)


def _vec(scale: torch.Tensor, n: int) -> torch.Tensor:
    flat = scale.reshape(-1).float()
    return flat.expand(n).contiguous() if flat.numel() == 1 else flat.contiguous()


def stash_hook(a, b, scale_a, scale_b, out_dtype, bias):  # noqa: ANN001
    """Dispatcher stash hook: when ``b`` is the qkv / out / fc2 weight of the running block (and the dispatcher runs
    the two-pass level), keep the fp32 product and return an uninitialised placeholder."""
    scope = _scope()
    if scope is None or out_dtype is not torch.bfloat16 or fp8_gemm._state.get("fused"):
        return None
    site = scope.want.pop(_sites_key(b), None)
    if site is None:
        return None
    scope.flush(f"a {site} GEMM arrived before the earlier stash was consumed")
    M, N = a.shape[0], b.shape[1]
    ph = torch.empty((M, N), device=a.device, dtype=out_dtype)
    scope.pending[site] = Stash(fp8_gemm.product_fp32(a, b), _vec(scale_a, M), _vec(scale_b, N), bias, ph)
    _stats["stash"] += 1
    return ph


def _sites_key(w: torch.Tensor) -> tuple:
    return w.data_ptr(), tuple(w.shape)


def set_fused(site: str, fn: Callable | None) -> None:
    """Register the fused consumer of ``site``: ``fn(stash, *args, **kwargs)`` returns the consumer's result computed
    from the stash, or None when it cannot take the call (the stash is then materialised and the stock consumer
    runs).  ``None`` removes it."""
    if site not in SITES:
        raise ValueError(f"unknown consumer site {site!r}")
    registry = _state["fused"]
    if fn is None:
        registry.pop(site, None)
    else:
        registry[site] = fn


def make_consumer_wrapper(site: str, orig):  # noqa: ANN001,ANN201
    """The wrapper of a site's consumer: the fused consumer on the site's stash when one is registered and takes the
    call, otherwise the stash materialised and the stock consumer."""
    @functools.wraps(orig)
    def consumer(*args, **kwargs):  # noqa: ANN002,ANN003,ANN202
        scope = _scope()
        st = scope.claim(site) if scope is not None else None
        if st is None:
            return orig(*args, **kwargs)
        fused = None if site in _state["disabled"] else _state["fused"].get(site)
        result = fused(st, *args, **kwargs) if fused is not None else None
        if result is not None:
            scope.settle(site)
            _stats["fused"] += 1
            return result
        scope.flush(f"{site}: no fused consumer took the call")
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
    v = ph[:, v0:].view(T, num_kv_heads, head_dim)
    if T and head_dim == 128 and x32.shape[1] == v0 + num_kv_heads * head_dim:
        # q, k and the v columns' scale pass in one launch
        oq, ok = ops.scale_qk_norm_rope(x32, sa, sb, bias, num_heads, num_kv_heads, q_weight.contiguous(),
                                        k_weight.contiguous(), rope_table, eps, v_out=v)
        return oq, ok, v
    oq, ok = ops.scale_qk_norm_rope(x32, sa, sb, bias, num_heads, num_kv_heads, q_weight.contiguous(),
                                    k_weight.contiguous(), rope_table, eps)
    if T:
        ops.scale_bias_cast(x32[:, v0:], sa, sb[v0:], None if bias is None else bias[v0:], torch.bfloat16,
                            out=ph[:, v0:])
    return oq, ok, v


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


# ---- when a fused consumer may take a call -------------------------------------------------------------------------
# Each rule is (reason, predicate that is True when the call is acceptable); the first failing rule names the reason.

def _first_failure(rules) -> str | None:  # noqa: ANN001
    for reason, ok in rules:
        if not ok():
            return reason
    return None


def _same_cuda_device(*ts: torch.Tensor) -> bool:
    dev = ts[0].device
    return dev.type == "cuda" and all(isinstance(t, torch.Tensor) and t.device == dev for t in ts)


def _is_view_of(x: torch.Tensor, base: torch.Tensor) -> bool:
    return x.data_ptr() == base.data_ptr() and x.stride() == base.stride()


def qk_mismatch(st: Stash, q, k, q_weight, k_weight, rope_table, head_dim, rotary_dim, interleaved) -> str | None:  # noqa: ANN001
    """None when (q, k) are exactly the q/k views of the stash's placeholder and the kernel takes the call
    (half-split, head_dim 128, rotary 96), else the reason."""
    ph, x32 = st.ph, st.x32

    def ranks():
        return q.dim() == 3 and k.dim() == 3 and q.dtype == k.dtype == torch.bfloat16

    def shapes():
        T, H, D = q.shape
        Hk = k.shape[1]
        return T > 0 and ph.dim() == 2 and ph.shape[0] == T and k.shape == (T, Hk, D) and ph.shape[1] == (H + 2 * Hk) * D

    def views():
        T, H, D = q.shape
        Hk = k.shape[1]
        return (_is_view_of(q, ph[:, :H * D].view(T, H, D))
                and _is_view_of(k, ph[:, H * D:(H + Hk) * D].view(T, Hk, D)))

    def rotary():
        rot = rope_table.shape[-1] if rope_table.dim() == 2 else -1
        return (rot == ROTARY_DIM and rotary_dim in (None, rot) and tuple(rope_table.shape) == (q.shape[0], rot)
                and rope_table.stride(1) == 1)

    def tables():
        D = q.shape[-1]
        return (rope_table.dtype in (torch.bfloat16, torch.float32) and q_weight.shape == (D,) and k_weight.shape == (D,)
                and q_weight.dtype == k_weight.dtype == torch.bfloat16)

    return _first_failure((
        ("interleaved", lambda: not interleaved),
        ("q / k are not bf16 [T, heads, head_dim]", ranks),
        ("shapes", shapes),
        ("stash not dense", lambda: ph.is_contiguous() and x32.is_contiguous() and x32.shape == ph.shape),
        ("q / k do not view the stashed qkv output", views),
        ("head_dim", lambda: q.shape[-1] == HEAD_DIM and head_dim in (None, HEAD_DIM)),
        ("rotary", rotary),
        ("norm weights or rope table of another shape or type", tables),
        ("device", lambda: _same_cuda_device(x32, q_weight, k_weight, rope_table)),
    ))


def _row_tables_ok(H: int, tables) -> bool:  # noqa: ANN001
    """gate / shift / scale rows the kernels take: bf16 [B > 0, H] with unit column stride, 16-byte aligned rows."""
    return all(t.dim() == 2 and t.stride(1) == 1 and t.dtype == torch.bfloat16 and t.shape[1] == H and t.shape[0] > 0
               and (t.shape[0] == 1 or t.stride(0) % 8 == 0) and t.data_ptr() % 16 == 0 for t in tables)


def rows_mismatch(st: Stash, x: torch.Tensor, branch: torch.Tensor, *others: torch.Tensor) -> str | None:
    """None when ``branch`` is exactly the stash's placeholder and ``x`` (the residual) a contiguous bf16 tensor of the
    same shape on the same device as the other operands (gate / shift / scale rows, then the indices)."""
    ph, x32 = st.ph, st.x32
    tables, idx = others[:-1], others[-1]
    return _first_failure((
        ("the branch is not the stashed output", lambda: _is_view_of(branch, ph) and branch.shape == ph.shape),
        ("the residual is not a dense bf16 twin of it", lambda: x.dim() == 2 and x.shape == ph.shape
         and x.dtype == torch.bfloat16
         and x.is_contiguous() and ph.is_contiguous() and x32.is_contiguous() and x32.shape == ph.shape),
        ("no rows", lambda: x.shape[0] > 0),
        ("width", lambda: x.shape[1] % 8 == 0 and x.shape[1] <= 8192),
        ("modulation tables the kernel cannot index", lambda: _row_tables_ok(x.shape[1], tables)),
        ("indices", lambda: idx.dim() == 1 and idx.shape[0] == x.shape[0] and idx.dtype in (torch.int32, torch.int64)),
        ("device", lambda: _same_cuda_device(x, x32, *others)),
    ))


class FusedConsumer:
    """The fused consumer of one site: ``mismatch(st, *args, **kwargs)`` says why it cannot take a call (None: it can);
    ``signature`` keys the once-per-process self-check, which runs ``sample_fused(st, r, ...)`` against
    ``sample_stock(st, r, ...)`` on the first r rows; ``run(st, ...)`` computes the call."""

    def __init__(self, site: str, mismatch, signature, sample_fused, sample_stock, run):  # noqa: ANN001
        self.site = site
        self.mismatch, self.signature = mismatch, signature
        self.sample_fused, self.sample_stock, self.run = sample_fused, sample_stock, run

    def __call__(self, st: Stash, *args, **kwargs):  # noqa: ANN002,ANN003,ANN204
        reason = self.mismatch(st, *args, **kwargs)
        if reason is not None:
            _notes.once(f"{self.site}-{reason}", "%s consumer not fused (%s)", self.site, reason)
            return None
        r = min(_SELFCHECK_ROWS, st.ph.shape[0])
        key = (self.site,) + self.signature(st, *args, **kwargs)
        if not _sites.checked(_state, _stats, _notes, key, lambda: self.sample_fused(st, r, *args, **kwargs),
                              lambda: self.sample_stock(st, r, *args, **kwargs)):
            return None
        out = self.run(st, *args, **kwargs)
        _stats["fused_" + self.site] += 1
        return out


def _heads(q, k):  # noqa: ANN001,ANN202
    return q.shape[1], k.shape[1], q.shape[-1]


def make_fused_qk(orig):  # noqa: ANN001,ANN201
    """The qkv site's fused consumer (registered by ``install``): ``fused_qk_norm_rope``'s arguments after the stash."""
    def mismatch(st, q, k, q_weight, k_weight, rope_table, eps, *, head_dim=None, rotary_dim=None, interleaved=False):  # noqa: ANN001,ANN202
        return qk_mismatch(st, q, k, q_weight, k_weight, rope_table, head_dim, rotary_dim, interleaved)

    def signature(st, q, k, q_weight, k_weight, rope_table, eps, **_):  # noqa: ANN001,ANN202,ANN003
        return tuple(st.ph.shape[1:]), rope_table.dtype

    def sample_fused(st, r, q, k, q_weight, k_weight, rope_table, eps, **_):  # noqa: ANN001,ANN202,ANN003
        return qk_norm_rope_fused(st.rows(r), *_heads(q, k), q_weight, k_weight, rope_table[:r], eps)

    def sample_stock(st, r, q, k, q_weight, k_weight, rope_table, eps, **kw):  # noqa: ANN001,ANN202,ANN003
        H, Hk, D = _heads(q, k)
        flat = st.rows(r).materialize()
        qs, ks, vs = flat[:, :H * D], flat[:, H * D:(H + Hk) * D], flat[:, (H + Hk) * D:]
        oq, ok = orig(qs.view(r, H, D), ks.view(r, Hk, D), q_weight, k_weight, rope_table[:r], eps, **kw)
        return oq, ok, vs.view(r, Hk, D)

    def run(st, q, k, q_weight, k_weight, rope_table, eps, **_):  # noqa: ANN001,ANN202,ANN003
        return qk_norm_rope_fused(st, *_heads(q, k), q_weight, k_weight, rope_table, eps)[:2]

    return FusedConsumer("qkv", mismatch, signature, sample_fused, sample_stock, run)


def _norm_weight_ok(weight: torch.Tensor, residual: torch.Tensor) -> bool:
    return (weight.shape == (residual.shape[1],) and weight.dtype == torch.bfloat16 and weight.is_contiguous()
            and weight.device == residual.device and weight.data_ptr() % 16 == 0)


def make_fused_gate_rms(orig):  # noqa: ANN001,ANN201
    """The out site's fused consumer: ``indexed_gate_rms_norm_scale_shift``'s arguments after the stash."""
    def mismatch(st, residual, gate, branch, weight, shift, scale, indices, eps):  # noqa: ANN001,ANN202
        reason = rows_mismatch(st, residual, branch, gate, shift, scale, indices)
        return reason if reason is not None or _norm_weight_ok(weight, residual) else "norm weight"

    def signature(st, residual, gate, branch, weight, *_):  # noqa: ANN001,ANN202,ANN002
        return tuple(residual.shape[1:]), gate.dtype, weight.dtype

    def sample_fused(st, r, residual, gate, branch, weight, shift, scale, indices, eps):  # noqa: ANN001,ANN202
        return gate_rms_fused(st.rows(r), residual[:r], gate, weight, shift, scale, indices[:r], eps)

    def sample_stock(st, r, residual, gate, branch, weight, shift, scale, indices, eps):  # noqa: ANN001,ANN202
        return orig(residual[:r], gate, st.rows(r).materialize(), weight, shift, scale, indices[:r], eps)

    def run(st, residual, gate, branch, weight, shift, scale, indices, eps):  # noqa: ANN001,ANN202
        return gate_rms_fused(st, residual, gate, weight, shift, scale, indices, eps)

    return FusedConsumer("out", mismatch, signature, sample_fused, sample_stock, run)


def make_fused_gate(orig):  # noqa: ANN001,ANN201
    """The fc2 site's fused consumer: ``indexed_gate``'s arguments after the stash."""
    def mismatch(st, x, gate, other, indices):  # noqa: ANN001,ANN202
        return rows_mismatch(st, x, other, gate, indices)

    def signature(st, x, gate, other, indices):  # noqa: ANN001,ANN202
        return tuple(x.shape[1:]), gate.dtype

    def sample_fused(st, r, x, gate, other, indices):  # noqa: ANN001,ANN202
        return (gate_fused(st.rows(r), x[:r].contiguous(), gate, indices[:r], reuse_placeholder=False),)

    def sample_stock(st, r, x, gate, other, indices):  # noqa: ANN001,ANN202
        return (orig(x[:r].contiguous(), gate, st.rows(r).materialize(), indices[:r]),)

    def run(st, x, gate, other, indices):  # noqa: ANN001,ANN202
        return gate_fused(st, x, gate, indices)

    return FusedConsumer("fc2", mismatch, signature, sample_fused, sample_stock, run)


FUSED_FACTORIES = {"qkv": make_fused_qk, "out": make_fused_gate_rms, "fc2": make_fused_gate}


# ---- the block scope -------------------------------------------------------------------------------------------------

def _stashable(site: str, layer, lora_types) -> str | None:  # noqa: ANN001
    """Why ``site``'s GEMM output cannot be replaced by a stash (None: it can): on top of the shared layer rules, the
    weight must be the dense FP8 [K, N] matrix the dispatcher sees (no padded output columns)."""
    why = _sites.layer_refusal(site, layer, lora_types)
    if why is not None:
        return why
    w = getattr(layer, "weight", None)
    width = int(getattr(layer, "output_size_per_partition", 0) or 0)
    dense = isinstance(w, torch.Tensor) and w.dtype == torch.float8_e4m3fn and w.dim() == 2 and w.shape[1] == width
    return None if dense else f"{site}: its weight is not a dense e4m3 [K, {width}] matrix"


def block_plan(block, sites, lora_types=()) -> tuple[dict | None, str]:  # noqa: ANN001
    """The weights of this block whose GEMMs may be stashed, as {weight key: site}, or (None, why not).  Every site
    still enabled must qualify, or the block runs stock."""
    if _sites.tracing():
        return None, "inside a torch.compile trace"
    layers = {site: _sites.site_layer(block, site) for site in sites if site not in _state["disabled"]}
    refusals = [why for why in (_stashable(site, layer, lora_types) for site, layer in layers.items()) if why]
    if refusals:
        return None, refusals[0]
    want = {_sites_key(layer.weight): site for site, layer in layers.items()}
    return (want or None), "every site is disabled"


def make_block_forward(orig_forward, sites, lora_types=()):  # noqa: ANN001,ANN201
    """Run a DiT block's forward inside a ConsumerScope (``_sites.block_scope``: thread-local, nested blocks restore
    the outer scope, a stash left waiting at the end is computed after all)."""
    @functools.wraps(orig_forward)
    def forward(self, *args, **kwargs):  # noqa: ANN001,ANN202
        want, why = block_plan(self, sites, lora_types)
        if want is None:
            _notes.once("plan-" + why, "%s: this block's consumers run stock", why)
            return orig_forward(self, *args, **kwargs)
        with _sites.block_scope(_tls, ConsumerScope(want)):
            return orig_forward(self, *args, **kwargs)

    forward._h3_tp2_amd_consumer = True
    return forward


def parse_sites(value: str | None) -> tuple[str, ...]:
    """"1"/"all" = every site; a comma list of qkv,out,fc2; empty/"0"/"off" = none."""
    return _sites.parse_site_list(value, SITES)


def _lora_base_types() -> tuple:
    try:
        from vllm.lora.layers import BaseLayerWithLoRA  # noqa: PLC0415
    except ImportError:
        return ()
    return (BaseLayerWithLoRA,)


def install(sites=SITES, tr=None, *, lora_types=None, fused: bool = True, check_source: bool = True,  # noqa: ANN001
            reviewed: dict | None = None, modules: dict | None = None) -> list[str]:
    """Wrap the block forward and the sites' consumers in the transformer module ``tr`` and register the stash hook;
    with ``fused`` also the fused consumer kernels of the sites.  Needs the dispatcher's two-pass level (at the
    default level there is no fp32 product to stash).  With ``check_source`` a site is wired only when the upstream
    functions it relies on fingerprint to the reviewed sources (``_drift``; ``reviewed`` / ``modules`` override the
    table and the upstream modules)."""
    chosen = tuple(site for site in SITES if site in sites)
    if not chosen:
        return []
    two_pass = fp8_gemm._state.get("level") == "tensor32" and not fp8_gemm._state.get("fused")
    if not two_pass:
        logger.warning("h3_tp2_amd fp8 consumers: needs the dispatcher's two-pass level; skipped")
        return []
    from . import fp8_hip  # noqa: PLC0415
    if fp8_hip.route in fp8_gemm._routers:
        # the block router computes its sites in bf16 ahead of the stash hook, so their consumers stay stock
        # (h3_tp2/fp8_consumers.py:870-877)
        routed = [site for site in chosen if site in fp8_hip.SITES]
        chosen = tuple(site for site in chosen if site not in fp8_hip.SITES)
        if routed:
            logger.warning("h3_tp2_amd fp8 consumers: the block router computes %s in bf16, so those consumers stay "
                           "stock; fused sites: %s", ", ".join(routed), ", ".join(chosen) or "none")
        if not chosen:
            return []
    if tr is None:
        from vllm_omni.diffusion.models.minimax_h3 import minimax_h3_transformer as tr  # noqa: PLC0415
    block_cls = tr.MiniMaxH3DiTBlock
    if getattr(block_cls.forward, "_h3_tp2_amd_consumer", False):
        return list(_state["sites"])
    if check_source:
        chosen = _drift.keep_sites("consumers", chosen, tr, _notes, reviewed, modules)
        if not chosen:
            return []
    for site in chosen:
        stock = getattr(tr, CONSUMERS[site])
        setattr(tr, CONSUMERS[site], make_consumer_wrapper(site, stock))
        if fused:
            set_fused(site, FUSED_FACTORIES[site](stock))
    block_cls.forward = make_block_forward(block_cls.forward, chosen,
                                           _lora_base_types() if lora_types is None else lora_types)
    fp8_gemm.set_stash_hook(stash_hook)
    _state["sites"] = chosen
    return list(chosen)


def stats() -> dict:
    return dict(_stats)
