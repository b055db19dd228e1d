"""Block router of the FP8 GEMM dispatcher: the running DiT block's qkv / out / fc1 GEMMs straight to kernel 2.

The counterpart of the reference's h3_tp2/fp8_cutlass.py routing (``route`` :134-159, ``block_want`` :252-263,
``make_block_forward`` :266-282, ``install_sites`` :285-294, ``selfcheck`` / ``probe`` :196-249, ``_verify``
:168-182).  While a block's forward runs, the router knows that block's FP8 weights by (data pointer, shape); a
dispatcher-eligible GEMM on one of them is computed here, ahead of the stash hooks, so its consumer receives an
ordinary bf16 tensor.  Every other GEMM goes on through the dispatcher.

Unlike the reference's DSL kernel, kernel 2 takes fp16 outputs, a bias and M = 0, so the router declines only calls
whose operands are not 16-byte aligned.  A launch error disables the router for the process (one warning) and the
call continues through the dispatcher; ``H3_TP2_AMD_VERIFY=1`` (diagnosis, slow) compares every routed output with
the two-pass form on the same operands and logs differences.
"""
from __future__ import annotations

import functools
import logging
import os
import threading
from typing import Any

import torch

from . import fp8_gemm

logger = logging.getLogger("h3_tp2_amd.fp8_hip")

SITES = ("qkv", "out", "fc1")
_ALIGN = 16

_tls = threading.local()   # want: {(weight data_ptr, weight shape): site} of the block whose forward is running
_state: dict[str, Any] = {"ok": False, "reason": "not probed"}
_stats = {"hip": 0, "fallthrough": 0, "verify_calls": 0, "verify_mismatch": 0}
_warned: set = set()
_VERIFY = os.environ.get("H3_TP2_AMD_VERIFY", "0").strip() == "1"


def _warn_once(key: str, msg: str, *args: Any) -> None:
    if key not in _warned:
        _warned.add(key)
        logger.warning("h3_tp2_amd fp8 router: " + msg, *args)


def _aligned(*ts: torch.Tensor) -> bool:
    return all(t.data_ptr() % _ALIGN == 0 for t in ts)


def scaled_mm(a, b, scale_a, scale_b, out_dtype, bias=None):  # noqa: ANN001,ANN201
    """Kernel 2 for one dispatcher-eligible call, or None when it cannot take it (the dispatch continues)."""
    if not _state["ok"] or not a.is_cuda:
        return None
    if not _aligned(a, b):
        return None
    return fp8_gemm.scaled_mm_fused(a, b, scale_a, scale_b, out_dtype, bias)


def route(a, b, scale_a, scale_b, out_dtype, bias):  # noqa: ANN001,ANN201
    """Dispatcher router (runs before the stash hooks): kernel 2 for the running block's qkv / out / fc1 GEMMs."""
    want = getattr(_tls, "want", None)
    if not want:
        return None
    site = want.get((b.data_ptr(), tuple(b.shape)))
    if site is None:
        return None
    try:
        y = scaled_mm(a, b, scale_a, scale_b, out_dtype, bias)
    except Exception as exc:  # noqa: BLE001  (the dispatcher's own path takes this call and the later ones)
        logger.warning("h3_tp2_amd fp8 router: launch failed (%s: %s); router off for this process",
                       type(exc).__name__, exc)
        _state.update(ok=False, reason=f"launch failed: {type(exc).__name__}")
        y = None
    if y is None:
        _stats["fallthrough"] += 1
        _warn_once("ft-" + site, "%s GEMM M=%d N=%d not taken (router off or unaligned operands)",
                   site, a.shape[0], b.shape[1])
        return None
    _stats["hip"] += 1
    if _VERIFY:
        _verify(site, a, b, scale_a, scale_b, out_dtype, bias, y)
    return y


def _verify(site, a, b, scale_a, scale_b, out_dtype, bias, y) -> None:  # noqa: ANN001
    ref = fp8_gemm.scaled_mm_tensor32(a, b, scale_a, scale_b, out_dtype, bias)
    nd = int((y.view(torch.int16) != ref.view(torch.int16)).sum())
    _stats["verify_calls"] += 1
    if nd:
        _stats["verify_mismatch"] += 1
        if _stats["verify_mismatch"] <= 20:
            logger.warning("h3_tp2_amd fp8 router VERIFY: %s M=%d N=%d K=%d: %d elements differ from two-pass",
                           site, a.shape[0], b.shape[1], a.shape[1], nd)


def probe(device="cuda") -> bool:  # noqa: ANN001
    """The dispatcher's install check, once per process; the router serves only when it passed."""
    try:
        bad = fp8_gemm.selfcheck(device)
    except Exception as exc:  # noqa: BLE001
        bad = [f"{type(exc).__name__}: {exc}"]
    if bad:
        _state.update(ok=False, reason="install check failed on " + "; ".join(bad))
        return False
    _state.update(ok=True, reason="install check passed")
    return True


def block_want(block, sites=SITES) -> dict:  # noqa: ANN001
    """{(weight data_ptr, weight shape): site} for this block's FP8 qkv / out / fc1 weights."""
    attn = getattr(block, "attn", None)
    mlp = getattr(block, "mlp", None)
    layers = {"qkv": getattr(attn, "qkv_proj", None), "out": getattr(attn, "out_proj", None),
              "fc1": getattr(mlp, "fc1", None), "fc2": getattr(mlp, "fc2", None)}
    want = {}
    for site in sites:
        w = getattr(layers.get(site), "weight", None)
        if isinstance(w, torch.Tensor) and w.dtype == torch.float8_e4m3fn and w.dim() == 2:
            want[(w.data_ptr(), tuple(w.shape))] = site
    return want


def make_block_forward(orig_forward, sites=SITES):  # noqa: ANN001,ANN201
    """Wrap a DiT block's forward so that the router knows the block's weights while it runs (thread-local, nested
    forwards restore the outer block's set)."""
    @functools.wraps(orig_forward)
    def forward(self, *args, **kwargs):  # noqa: ANN001,ANN202
        try:
            if torch.compiler.is_compiling():
                return orig_forward(self, *args, **kwargs)
        except AttributeError:
            pass
        prev = getattr(_tls, "want", None)
        _tls.want = block_want(self, sites)
        try:
            return orig_forward(self, *args, **kwargs)
        finally:
            _tls.want = prev

    forward._h3_tp2_amd_router = True
    return forward


def install_sites(tr=None, sites=SITES, check: bool = True) -> bool:  # noqa: ANN001
    """Register the router with the dispatcher and wrap ``MiniMaxH3DiTBlock.forward`` of the transformer module ``tr``
    (default: vLLM-Omni's MiniMax H3).  With ``check`` the install check runs first; on failure nothing is wired."""
    if tr is None:
        from vllm_omni.diffusion.models.minimax_h3 import minimax_h3_transformer as tr  # noqa: PLC0415
    if check and not probe():
        logger.warning("h3_tp2_amd fp8 router: unavailable (%s)", _state["reason"])
        return False
    if not check:
        _state.update(ok=True, reason="install check skipped")
    cls = tr.MiniMaxH3DiTBlock
    if not getattr(cls.forward, "_h3_tp2_amd_router", False):
        cls.forward = make_block_forward(cls.forward, sites)
    fp8_gemm.set_router(route)
    return True


def stats() -> dict:
    return dict(_stats)
