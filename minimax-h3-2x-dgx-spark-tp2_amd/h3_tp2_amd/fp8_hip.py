"""Block router of the FP8 GEMM dispatcher: the running DiT block's qkv / out / fc1 GEMMs straight to kernel 2.

The counterpart of the reference's h3_tp2/fp8_cutlass.py routing surface (``route`` :134-159, ``block_want``
:252-263, ``make_block_forward`` :266-282, ``install_sites`` :285-294, ``probe`` :228-249, ``_verify`` :168-182): the
same names and call contract, a design of its own.

* While a block's forward runs, a routing scope (``_routing``) publishes the block's FP8 weights in the thread-local
  ``_tls.want`` as {(data pointer, shape): site}; nested forwards see their own block and restore the outer one.
* The dispatcher calls ``route`` for every eligible GEMM before its stash hooks.  A GEMM on one of the published weights
  is computed here by kernel 2 and its consumer receives an ordinary bf16 tensor; any other GEMM is declined (None) and
  goes on through the dispatcher.
* Kernel 2 takes fp16 outputs, a bias and M = 0, unlike the reference's DSL kernel, so the router declines only
  operands that are not 16-byte aligned.  A launch error switches the router off for the process (one warning) and the
  call goes on through the dispatcher.  ``H3_TP2_AMD_VERIFY=1`` (diagnosis, slow) compares every routed output with the
  two-pass form on the same operands and logs the differences.
"""
from __future__ import annotations

import contextlib
import functools
import logging
import os
import threading
from typing import Any

import torch

from . import fp8_gemm

logger = logging.getLogger("h3_tp2_amd.fp8_hip")

SITES = ("qkv", "out", "fc1")
# where each site's linear layer hangs off a MiniMax H3 DiT block
SITE_LAYERS = {"qkv": ("attn", "qkv_proj"), "out": ("attn", "out_proj"), "fc1": ("mlp", "fc1"), "fc2": ("mlp", "fc2")}
_ALIGN = 16

_tls = threading.local()   # want: {(weight data_ptr, weight shape): site} of the block whose forward is running
_state: dict[str, Any] = {"ok": False, "reason": "not probed"}
_stats = {"hip": 0, "fallthrough": 0, "verify_calls": 0, "verify_mismatch": 0}
_reported: set = set()
_VERIFY = os.environ.get("H3_TP2_AMD_VERIFY", "0").strip() == "1"


def _report(key: str, msg: str, *args: Any) -> None:
    """Log ``msg`` the first time ``key`` is seen in this process."""
    if key in _reported:
        return
    _reported.add(key)
    logger.warning("h3_tp2_amd fp8 router: " + msg, *args)


def weight_key(w: torch.Tensor) -> tuple:
    """The identity under which a weight is published: its storage address and its shape."""
    return w.data_ptr(), tuple(w.shape)


def _site_weight(block, site: str):  # noqa: ANN001,ANN202
    """The FP8 weight of ``site``'s layer in ``block`` (2-D e4m3fn), or None."""
    owner, name = SITE_LAYERS[site]
    w = getattr(getattr(getattr(block, owner, None), name, None), "weight", None)
    ok = isinstance(w, torch.Tensor) and w.dtype == torch.float8_e4m3fn and w.dim() == 2
    return w if ok else None


def block_want(block, sites=SITES) -> dict:  # noqa: ANN001
    """The block's FP8 qkv / out / fc1 weights as the router looks them up: weight key -> site."""
    found = ((site, _site_weight(block, site)) for site in sites)
    return {weight_key(w): site for site, w in found if w is not None}


def scaled_mm(a, b, scale_a, scale_b, out_dtype, bias=None):  # noqa: ANN001,ANN201
    """Kernel 2 for one dispatcher-eligible call, or None when the router cannot take it."""
    usable = _state["ok"] and a.is_cuda and a.data_ptr() % _ALIGN == 0 and b.data_ptr() % _ALIGN == 0
    return fp8_gemm.scaled_mm_fused(a, b, scale_a, scale_b, out_dtype, bias) if usable else None


def _switch_off(exc: Exception) -> None:
    _state.update(ok=False, reason=f"launch failed: {type(exc).__name__}")
    logger.warning("h3_tp2_amd fp8 router: launch failed (%s: %s); router off for this process",
                   type(exc).__name__, exc)


def route(a, b, scale_a, scale_b, out_dtype, bias):  # noqa: ANN001,ANN201
    """Dispatcher router (runs before the stash hooks): kernel 2 for the running block's qkv / out / fc1 GEMMs."""
    site = (getattr(_tls, "want", None) or {}).get(weight_key(b))
    if site is None:
        return None
    y = None
    try:
        y = scaled_mm(a, b, scale_a, scale_b, out_dtype, bias)
    except Exception as exc:  # noqa: BLE001  (the dispatcher's own path takes this call and the later ones)
        _switch_off(exc)
    if y is None:
        _stats["fallthrough"] += 1
        _report("declined-" + site, "%s GEMM M=%d N=%d not taken (router off or unaligned operands)",
                site, a.shape[0], b.shape[1])
        return None
    _stats["hip"] += 1
    if _VERIFY:
        _verify(site, a, b, scale_a, scale_b, out_dtype, bias, y)
    return y


def _verify(site, a, b, scale_a, scale_b, out_dtype, bias, y) -> None:  # noqa: ANN001
    """Diagnosis: the routed output against the two-pass form of the same call, differences logged."""
    two_pass = fp8_gemm.scaled_mm_tensor32(a, b, scale_a, scale_b, out_dtype, bias)
    differ = int(torch.count_nonzero(y.view(torch.int16) != two_pass.view(torch.int16)))
    _stats["verify_calls"] += 1
    if not differ:
        return
    _stats["verify_mismatch"] += 1
    if _stats["verify_mismatch"] <= 20:
        logger.warning("h3_tp2_amd fp8 router VERIFY: %s M=%d N=%d K=%d: %d elements differ from two-pass",
                       site, a.shape[0], b.shape[1], a.shape[1], differ)


def probe(device="cuda") -> bool:  # noqa: ANN001
    """The dispatcher's install check, once per process; the router serves only when it passed."""
    try:
        failing = fp8_gemm.selfcheck(device)
    except Exception as exc:  # noqa: BLE001
        failing = [f"{type(exc).__name__}: {exc}"]
    _state["ok"] = not failing
    _state["reason"] = "install check passed" if not failing else "install check failed on " + "; ".join(failing)
    return _state["ok"]


@contextlib.contextmanager
def _routing(want: dict):
    """Publish ``want`` as the running block's weights for the duration; the enclosing block's set comes back after."""
    outer = getattr(_tls, "want", None)
    _tls.want = want
    try:
        yield
    finally:
        _tls.want = outer


def _tracing() -> bool:
    """True while torch.compile traces: the router stays out of traced graphs (the stock path is traced)."""
    is_compiling = getattr(getattr(torch, "compiler", None), "is_compiling", None)
    return bool(is_compiling and is_compiling())


def make_block_forward(orig_forward, sites=SITES):  # noqa: ANN001,ANN201
    """Wrap a DiT block's forward so that the router knows the block's weights while it runs."""
    @functools.wraps(orig_forward)
    def forward(self, *args, **kwargs):  # noqa: ANN001,ANN202
        if _tracing():
            return orig_forward(self, *args, **kwargs)
        with _routing(block_want(self, sites)):
            return orig_forward(self, *args, **kwargs)

    forward._h3_tp2_amd_router = True
    return forward


def install_sites(tr=None, sites=SITES, check: bool = True) -> bool:  # noqa: ANN001
    """Register the router with the dispatcher and wrap ``MiniMaxH3DiTBlock.forward`` of the transformer module ``tr``
    (default: vLLM-Omni's MiniMax H3).  With ``check`` the install check runs first; on failure nothing is wired."""
    if tr is None:
        from vllm_omni.diffusion.models.minimax_h3 import minimax_h3_transformer as tr  # noqa: PLC0415
    if check:
        if not probe():
            logger.warning("h3_tp2_amd fp8 router: unavailable (%s)", _state["reason"])
            return False
    else:
        _state.update(ok=True, reason="install check skipped")
    block = tr.MiniMaxH3DiTBlock
    if not getattr(block.forward, "_h3_tp2_amd_router", False):
        block.forward = make_block_forward(block.forward, sites)
    fp8_gemm.set_router(route)
    return True


def stats() -> dict:
    return dict(_stats)
