"""Source fingerprints of the upstream code the hook sites rely on: a site is wired only over the reviewed sources.

A fused site replaces an upstream function or relies on the dataflow of an upstream forward (fc1's output reaching
the MLP's activation, the norm's output reaching the QKV projection's quant, a GEMM's output reaching its consumer
before anything else reads it).  The per-shape self-checks cover the kernels' arithmetic, not that dataflow; if
upstream changes a forward, a stash could reach the wrong consumer unnoticed.  So every site names the upstream
functions it relies on (``NEEDS``), and ``install`` wires a site only when each of them fingerprints to the reviewed
value (``REVIEWED``): the sha256 (first 16 hex digits) of the function's source lines stripped of surrounding white
space, with empty lines, comment lines and decorator lines dropped.  A changed, missing or foreign-wrapped function
leaves the site stock, with a warning naming it.

The four functions the transformer module calls by name (``fused_qk_norm_rope``, ``indexed_gate``,
``indexed_gate_rms_norm_scale_shift``, ``rms_norm_indexed_scale_shift``) are fingerprinted in their upstream module,
and the transformer's binding must be that very function (h3_tp2/fp8_consumers.py:849-855, fp8_quant_fuse.py:891-892):
a wrapper installed there by someone else -- with ``functools.wraps`` or without -- is drift, since a fused site would
replace the call and drop what the wrapper does.  Only this library's own wrappers are seen through: functions whose
code lives in this package (``functools.wraps`` copies names and attributes, never the code object) that carry an
``_h3_tp2_amd*`` marker and say what they wrap in ``__wrapped__``.

``REVIEWED`` holds the fingerprints of vLLM-Omni v0.30.0 (commit a8576ccb7) and vLLM 0.30.0 -- the upstream the
reference's sites were reviewed against (h3_tp2/fp8_consumers.py:64-80, h3_tp2/fp8_quant_fuse.py:857-877); they are
facts about those sources under this normalisation, so they carry over unchanged.
"""
from __future__ import annotations

import hashlib
import inspect
import os
from typing import Any, Callable

_PKG_DIR = os.path.dirname(os.path.abspath(__file__))
WRAPPED = "wrapped"      # a by-name binding that is not the upstream function (nor this library's wrapper of it)

REVIEWED = {
    # vllm_omni/diffusion/models/minimax_h3/minimax_h3_transformer.py
    "attn_forward": "b2a25e0b45bea674",          # MiniMaxH3Attention.forward
    "block_forward": "c052863b435652b7",         # MiniMaxH3DiTBlock.forward
    "mlp_forward": "ac9fa6ab2762a4bb",           # MiniMaxH3MLP.forward
    "run_packed": "89368785eed0feec",            # MiniMaxH3Attention._run_packed_attention
    # vllm_omni/diffusion/layers/fused_qk_norm_rope.py
    "rms_norm_rope_kernel": "dde848323d52afbd",
    "launch_fused_rms_norm_rope": "06631d16d022e0ef",
    "fused_qk_norm_rope_impl": "dbc570960f4b3a99",
    "fused_qk_norm_rope": "38d2d10a3af2d594",
    "fused_cuda_supported": "979429af70cdbf7b",
    # vllm_omni/diffusion/layers/indexed_modulation.py
    "indexed_gate_kernel": "9273a7807bd876ab",
    "indexed_gate": "0c16c223345767c7",
    "gate_rms_kernel": "7d239874d6fcab35",
    "gate_rms": "b0d503b521d61c64",
    "rms_kernel": "b791a0e3dec74b2e",
    "rms": "373f4b3620d23b43",
    "launch_row_chunks": "9260a692db6402e3",
    # vllm_omni/diffusion/layers/activation.py, vllm_omni/diffusion/attention/layer.py
    "silu_forward_cuda": "cc7021d08b7cfd95",     # SiluAndMul.forward_cuda
    "attn_layer_forward": "101199f5a077548b",    # Attention.forward
    # vllm/model_executor/layers/linear.py, .../kernels/linear/scaled_mm/ScaledMMLinearKernel.py
    "col_forward": "af4d0eb5573d0dc6",           # ColumnParallelLinear.forward
    "row_forward": "693d179dcadc13ff",           # RowParallelLinear.forward
    "apply_weights": "54ad02f4f844454d",         # FP8ScaledMMLinearKernel.apply_weights
}

# the upstream functions each site relies on, per protocol
NEEDS = {
    "consumers": {
        "qkv": ("block_forward", "attn_forward", "rms_norm_rope_kernel", "launch_fused_rms_norm_rope",
                "fused_qk_norm_rope_impl", "fused_qk_norm_rope", "fused_cuda_supported"),
        "out": ("block_forward", "attn_forward", "gate_rms_kernel", "gate_rms", "launch_row_chunks"),
        "fc2": ("block_forward", "mlp_forward", "indexed_gate_kernel", "indexed_gate", "launch_row_chunks"),
    },
    "producers": {
        "qkv": ("block_forward", "attn_forward", "rms_kernel", "rms", "launch_row_chunks", "col_forward",
                "apply_weights"),
        "fc1": ("block_forward", "mlp_forward", "gate_rms_kernel", "gate_rms", "launch_row_chunks", "col_forward",
                "apply_weights"),
        "fc2": ("block_forward", "mlp_forward", "silu_forward_cuda", "row_forward", "apply_weights"),
    },
    "mlp": {"fc1": ("mlp_forward",)},
}


def normalised_lines(src: str) -> list[str]:
    out = []
    for line in src.splitlines():
        text = line.strip()
        if text and text[0] not in "#@":
            out.append(text)
    return out


def fingerprint_source(src: str) -> str:
    return hashlib.sha256("\n".join(normalised_lines(src)).encode()).hexdigest()[:16]


def is_own_wrapper(fn: Any) -> bool:
    """True for a wrapper this library installed: its code is defined in this package, it carries an ``_h3_tp2_amd*``
    marker and names what it wraps in ``__wrapped__``."""
    code = getattr(fn, "__code__", None)
    if code is None or getattr(fn, "__wrapped__", None) is None:
        return False
    if os.path.dirname(os.path.abspath(code.co_filename)) != _PKG_DIR:
        return False
    return any(k.startswith("_h3_tp2_amd") for k in vars(fn))


def own_unwrap(fn: Any) -> Any:
    """``fn`` with this library's own wrappers taken off (any other wrapper stays)."""
    for _ in range(16):
        if not is_own_wrapper(fn):
            break
        fn = fn.__wrapped__
    return fn


def fingerprint(fn: Any) -> str | None:
    """The fingerprint of a function's source (a Triton kernel's ``fn``; as in the reference, ``inspect`` sees through
    functools.wraps wrappers of methods); None when its source cannot be read."""
    fn = getattr(fn, "fn", fn)
    try:
        return fingerprint_source(inspect.getsource(fn))
    except (OSError, TypeError):
        return None


def _bound(tr: Any, name: str, module: Any) -> Any:
    """The upstream function ``module.name`` when the transformer module ``tr`` calls exactly it (or this library's
    wrapper of it) under ``name``; WRAPPED when ``tr`` binds something else; None when either is absent."""
    upstream = getattr(module, name, None) if module is not None else None
    binding = getattr(tr, name, None)
    if upstream is None or binding is None:
        return None
    return upstream if own_unwrap(binding) is upstream else WRAPPED


def _attr(obj: Any, *path: str) -> Any:
    for name in path:
        obj = getattr(obj, name, None)
    return obj


def _upstream_modules() -> dict:
    """The vLLM / vLLM-Omni modules that hold the upstream functions (absent ones left out)."""
    found: dict[str, Any] = {}
    for key, name in (("qk", "vllm_omni.diffusion.layers.fused_qk_norm_rope"),
                      ("im", "vllm_omni.diffusion.layers.indexed_modulation"),
                      ("act", "vllm_omni.diffusion.layers.activation"),
                      ("attn_layer", "vllm_omni.diffusion.attention.layer"),
                      ("linear", "vllm.model_executor.layers.linear"),
                      ("smm", "vllm.model_executor.kernels.linear.scaled_mm.ScaledMMLinearKernel")):
        try:
            found[key] = __import__(name, fromlist=["_"])
        except ImportError:
            pass
    return found


def resolvers(tr: Any, modules: dict | None = None) -> dict[str, Callable[[], Any]]:
    """name -> a function returning the upstream object to fingerprint (None: absent), for the transformer module
    ``tr`` and the upstream modules (default: imported when present)."""
    m = _upstream_modules() if modules is None else modules
    return {
        "attn_forward": lambda: _attr(tr, "MiniMaxH3Attention", "forward"),
        "block_forward": lambda: _attr(tr, "MiniMaxH3DiTBlock", "forward"),
        "mlp_forward": lambda: _attr(tr, "MiniMaxH3MLP", "forward"),
        "run_packed": lambda: _attr(tr, "MiniMaxH3Attention", "_run_packed_attention"),
        "rms_norm_rope_kernel": lambda: _attr(m.get("qk"), "_rms_norm_rope_kernel"),
        "launch_fused_rms_norm_rope": lambda: _attr(m.get("qk"), "_launch_fused_rms_norm_rope"),
        "fused_qk_norm_rope_impl": lambda: _attr(m.get("qk"), "_fused_qk_norm_rope_impl"),
        # the functions the transformer module calls by name: the upstream module's own function, and the
        # transformer's binding must be it (any other wrapper there is drift)
        "fused_qk_norm_rope": lambda: _bound(tr, "fused_qk_norm_rope", m.get("qk")),
        "fused_cuda_supported": lambda: _attr(m.get("qk"), "_fused_cuda_supported"),
        "indexed_gate_kernel": lambda: _attr(m.get("im"), "_indexed_gate_kernel"),
        "indexed_gate": lambda: _bound(tr, "indexed_gate", m.get("im")),
        "gate_rms_kernel": lambda: _attr(m.get("im"), "_indexed_gate_rms_norm_scale_shift_kernel"),
        "gate_rms": lambda: _bound(tr, "indexed_gate_rms_norm_scale_shift", m.get("im")),
        "rms_kernel": lambda: _attr(m.get("im"), "_rms_norm_indexed_scale_shift_kernel"),
        "rms": lambda: _bound(tr, "rms_norm_indexed_scale_shift", m.get("im")),
        "launch_row_chunks": lambda: _attr(m.get("im"), "_launch_row_chunks"),
        "silu_forward_cuda": lambda: _attr(m.get("act"), "SiluAndMul", "forward_cuda"),
        "attn_layer_forward": lambda: _attr(m.get("attn_layer"), "Attention", "forward"),
        "col_forward": lambda: _attr(m.get("linear"), "ColumnParallelLinear", "forward"),
        "row_forward": lambda: _attr(m.get("linear"), "RowParallelLinear", "forward"),
        "apply_weights": lambda: _attr(m.get("smm"), "FP8ScaledMMLinearKernel", "apply_weights"),
    }


def drifted(names, found: dict[str, Callable[[], Any]], reviewed: dict[str, str] | None = None) -> list[str]:  # noqa: ANN001
    """The names among ``names`` whose upstream function is absent or fingerprints otherwise than reviewed, each as
    "name: got (reviewed want)"."""
    table = REVIEWED if reviewed is None else reviewed
    out = []
    for name in names:
        obj = found[name]() if name in found else None
        got = WRAPPED if obj is WRAPPED else fingerprint(own_unwrap(obj)) if obj is not None else "absent"
        if got != table.get(name):
            out.append(f"{name}: {got} (reviewed {table.get(name)})")
    return out


def keep_sites(protocol: str, sites, tr: Any, notes, reviewed: dict[str, str] | None = None,  # noqa: ANN001
               modules: dict | None = None) -> tuple:
    """The sites of ``protocol`` whose upstream sources are the reviewed ones; the others are named in a warning."""
    found = resolvers(tr, modules)
    keep = []
    for site in sites:
        bad = drifted(NEEDS[protocol].get(site, ()), found, reviewed)
        if bad:
            notes.once(f"drift-{protocol}-{site}", "site %s skipped, upstream source differs from the reviewed one: %s",
                       site, "; ".join(bad))
        else:
            keep.append(site)
    return tuple(keep)
