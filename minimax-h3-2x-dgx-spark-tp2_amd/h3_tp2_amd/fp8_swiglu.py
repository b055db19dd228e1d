"""Fused FP8 gate/up GEMM + SwiGLU (+ per-token requant) for the DiT MLP on MI355X.

Mirrors the reference's h3_tp2/fp8_swiglu.py host surface -- ``scale_swiglu`` (:180-188), ``scale_swiglu_quant``
(:191-200), ``GemmOperands`` (:215-224), ``gemm_swiglu`` (:230-241), ``probe_gemm_swiglu`` (:258-284), ``_fc2_direct``
(:297-312), ``install`` / ``_install_on`` (:315-396) and ``_stash_hook`` (:399-421) -- with the compute on kernel 3:

* the MLP forward asks the dispatcher's stash hook for fc1's operands (thread-local request, as in the reference);
  fc1 returns an uninitialised placeholder and no GEMM runs at that point;
* level 1: kernel 3 computes gate and up for the same output columns from each A tile and applies the SwiGLU epilogue
  on the accumulators: bf16 h [M, F], then fc2 as usual;
* level 2: kernel 3 also reduces each row's max |h| and the quant tail writes fc2's e4m3 input and per-token scale;
  fc2 runs on them directly (vLLM's ``apply_scaled_mm``), its own quant is skipped.

The SwiGLU arithmetic (for each output column c): g, u = bf16(epilogue(acc)) of gate column c and up column F + c;
u = +0 where u == 0; s = bf16(g / (1 + exp(-g))) with a correctly rounded exp; h = bf16(s * u).
"""
from __future__ import annotations

import logging
import threading

import torch

from . import fp8_gemm, ops

logger = logging.getLogger("h3_tp2_amd.fp8_swiglu")

_tls = threading.local()
# gemm_swiglu: kernel 3 passed its install check (otherwise fc1's fp32 product is stashed and the standalone pass runs);
# fc2_kernel_cls: the class whose ``apply_scaled_mm`` takes fc2 on a pre-quantised input (vLLM's
# FP8ScaledMMLinearKernel, looked up lazily; a caller without vLLM sets it).
_state = {"gemm_swiglu": False, "level": 0, "fc2_kernel_cls": None}
_stats = {"fused": 0, "fused_quant": 0, "x32": 0, "stock": 0, "fc2_direct": 0, "fc2_redo": 0}


class GemmOperands:
    """Stashed in place of fc1's fp32 product: kernel 3 computes the product from the operands."""
    __slots__ = ("a", "b")

    def __init__(self, a: torch.Tensor, b: torch.Tensor):
        self.a, self.b = a, b

    @property
    def shape(self):  # noqa: ANN201
        return (self.a.shape[0], self.b.shape[1])


def scale_swiglu(x32: torch.Tensor, sa: torch.Tensor, sb: torch.Tensor, bias: torch.Tensor | None) -> torch.Tensor:
    """fp32 product [M, 2F] -> bf16 SwiGLU [M, F] (the stash form)."""
    return ops.scale_swiglu(x32, sa.reshape(-1), sb.reshape(-1), _bias(bias))


def scale_swiglu_quant(x32: torch.Tensor, sa: torch.Tensor, sb: torch.Tensor, bias: torch.Tensor | None):
    """fp32 product [M, 2F] -> SwiGLU -> per-token quant for fc2: (fp8 [M, F], fp32 scales [M, 1])."""
    return ops.scale_swiglu_quant(x32, sa.reshape(-1), sb.reshape(-1), _bias(bias))


def gemm_swiglu(a: torch.Tensor, b: torch.Tensor, sa: torch.Tensor, sb: torch.Tensor,
                bias: torch.Tensor | None) -> torch.Tensor:
    """fc1 + epilogue + SwiGLU in one kernel: bf16 [M, N/2] from fp8 a [M, K], b [K, N] (b.t() contiguous)."""
    return ops.gemm_swiglu(a, b.t(), sa.reshape(-1), sb.reshape(-1), _bias(bias))


def gemm_swiglu_quant(a: torch.Tensor, b: torch.Tensor, sa: torch.Tensor, sb: torch.Tensor,
                      bias: torch.Tensor | None):
    """fc1 + SwiGLU + per-token requant: (fp8 [M, N/2], fp32 scales [M, 1])."""
    return ops.gemm_swiglu_quant(a, b.t(), sa.reshape(-1), sb.reshape(-1), _bias(bias))


def _bias(bias):  # noqa: ANN001,ANN202
    return bias if bias is None or bias.dtype == torch.bfloat16 else bias.to(torch.bfloat16)


def probe_gemm_swiglu(device="cuda") -> bool:  # noqa: ANN001
    """Install check for kernel 3: on integer inputs (exact accumulators in any order) it must equal the raw product +
    standalone SwiGLU pass bit for bit, with and without the requant; on random inputs the two forms agree to the
    accumulation-order noise of one bf16 rounding."""
    try:
        g = torch.Generator(device="cpu").manual_seed(0)
        M, width, K = 200, 2 * 320, 512
        a = torch.randint(-4, 5, (M, K), generator=g).float().to(device).to(torch.float8_e4m3fn)
        w = torch.randint(-2, 3, (width, K), generator=g).float().to(device).to(torch.float8_e4m3fn)
        sa = (torch.rand(M, generator=g) * 0.01 + 1e-3).to(device)
        sb = (torch.rand(width, generator=g) * 0.01 + 1e-3).to(device)
        x32 = fp8_gemm.product_fp32(a, w.t())
        ok = torch.equal(gemm_swiglu(a, w.t(), sa, sb, None).view(torch.int16),
                         scale_swiglu(x32, sa, sb, None).view(torch.int16))
        q1, s1 = gemm_swiglu_quant(a, w.t(), sa, sb, None)
        q2, s2 = scale_swiglu_quant(x32, sa, sb, None)
        ok = ok and torch.equal(q1.view(torch.uint8), q2.view(torch.uint8)) and torch.equal(s1, s2)
        a = (torch.randn(M, K, generator=g) * 2).to(device).to(torch.float8_e4m3fn)
        w = (torch.randn(width, K, generator=g) * 0.5).to(device).to(torch.float8_e4m3fn)
        x32 = fp8_gemm.product_fp32(a, w.t())
        y = gemm_swiglu(a, w.t(), sa, sb, None).float()
        r = scale_swiglu(x32, sa, sb, None).float()
        ok = ok and bool(torch.isfinite(y).all()) and (y - r).abs().max().item() <= 1e-2 * r.abs().max().item() + 1e-5
        torch.cuda.synchronize(device)
        if not ok:
            logger.warning("h3_tp2_amd: fused FP8 GEMM + SwiGLU failed its install check; fc1 keeps the fp32 stash")
    except Exception as exc:  # noqa: BLE001
        logger.warning("h3_tp2_amd: fused FP8 GEMM + SwiGLU unavailable (%s); fc1 keeps the fp32 stash", exc)
        ok = False
    _state["gemm_swiglu"] = ok
    return ok


def _fc2_kernel_cls():  # noqa: ANN202
    cls = _state["fc2_kernel_cls"]
    if cls is not None:
        return cls
    try:
        from vllm.model_executor.kernels.linear.scaled_mm.ScaledMMLinearKernel import (  # noqa: PLC0415
            FP8ScaledMMLinearKernel)
    except ImportError:
        return None
    _state["fc2_kernel_cls"] = FP8ScaledMMLinearKernel
    return FP8ScaledMMLinearKernel


def _fc2_direct(fc2, q: torch.Tensor, scale: torch.Tensor, lead) -> torch.Tensor | None:  # noqa: ANN001
    """fc2 on the pre-quantised input through its own scaled-mm kernel (its ``apply_weights`` would quantise again).
    Only the plain case the model uses (tp 1, no bias, an FP8 scaled-mm kernel); otherwise None."""
    kcls = _fc2_kernel_cls()
    kernel = getattr(getattr(fc2, "quant_method", None), "fp8_linear", None)
    if kcls is None or not isinstance(kernel, kcls) or getattr(fc2, "tp_size", 1) != 1 \
            or getattr(fc2, "bias", None) is not None or getattr(fc2, "skip_bias_add", False):
        return None
    w, w_s, _, _ = kernel._get_layer_params(fc2)
    if w.shape[0] != q.shape[1]:
        return None
    return kernel.apply_scaled_mm(A=q, B=w, out_dtype=torch.bfloat16, As=scale, Bs=w_s, bias=None,
                                  output_shape=[*lead, w.shape[1]])


def _stash_hook(a, b, scale_a, scale_b, out_dtype, bias):  # noqa: ANN001
    """Dispatcher stash hook: when the MLP forward requested it, keep fc1's operands (or, without kernel 3, its fp32
    product) and return an uninitialised placeholder of the output's shape."""
    if not getattr(_tls, "stash_next", False) or out_dtype is not torch.bfloat16:
        return None
    M, N = a.shape[0], b.shape[1]
    expect = getattr(_tls, "expect_n", 0)
    if N % 2 or (expect and N != expect):              # padded fc1 (N != the logical width): the ordinary path
        _tls.stash_next = False
        return None
    sa, sb = fp8_gemm._vec_scales(scale_a, scale_b, M, N)
    if _state["gemm_swiglu"]:
        _tls.stash = (GemmOperands(a, b), sa, sb, bias)
    else:
        _tls.stash = (fp8_gemm.product_fp32(a, b), sa, sb, bias)
    _tls.stash_next = False
    return torch.empty((M, N), device=a.device, dtype=out_dtype)   # placeholder, never read


def _install_on(cls, *, level: int, lora_layer_type=()) -> bool:  # noqa: ANN001
    """Wrap ``cls.forward`` (an MLP with ``fc1``, ``act_fn``, ``fc2``); False when already wrapped."""
    if getattr(cls, "_h3_tp2_amd_swiglu", False):
        return False
    orig_forward = cls.forward
    fuse_quant = level >= 2

    def forward(self, x):  # noqa: ANN001,ANN202
        # A LoRA wrapper adds its delta to fc1's returned tensor (which the fused path discards) and level 2 bypasses
        # fc2's wrapper: such MLPs take the ordinary path.
        if lora_layer_type and (isinstance(self.fc1, lora_layer_type) or isinstance(self.fc2, lora_layer_type)):
            return orig_forward(self, x)
        _tls.stash_next = True
        _tls.stash = None
        _tls.expect_n = int(getattr(self.fc1, "output_size_per_partition", 0) or 0)
        stash = None
        try:
            hidden, _ = self.fc1(x)
            stash = _tls.stash
        finally:
            _tls.stash_next = False
            _tls.stash = None
            _tls.expect_n = 0
        if stash is None:
            _stats["stock"] += 1
            hidden = self.act_fn(hidden)
        else:
            lead = hidden.shape[:-1]
            del hidden                                   # the placeholder was never written
            x32, sa, sb, bias = stash
            del stash
            ops_in = isinstance(x32, GemmOperands)
            if fuse_quant:
                if ops_in:
                    q, scale = gemm_swiglu_quant(x32.a, x32.b, sa, sb, bias)
                    _stats["fused_quant"] += 1
                else:
                    q, scale = scale_swiglu_quant(x32, sa, sb, bias)
                    _stats["x32"] += 1
                del x32, sa, sb, bias
                out = _fc2_direct(self.fc2, q, scale, lead)
                if out is not None:
                    _stats["fc2_direct"] += 1
                    return out
                del q, scale
                # fc2 layout the direct call does not take: redo fc1 through the ordinary path (correct, slower)
                _stats["fc2_redo"] += 1
                hidden, _ = self.fc1(x)
                hidden = self.act_fn(hidden)
            elif ops_in:
                hidden = gemm_swiglu(x32.a, x32.b, sa, sb, bias).view(*lead, x32.shape[1] // 2)
                _stats["fused"] += 1
                del x32, sa, sb, bias
            else:
                hidden = scale_swiglu(x32, sa, sb, bias).view(*lead, x32.shape[1] // 2)
                _stats["x32"] += 1
                del x32, sa, sb, bias
        out, _ = self.fc2(hidden)
        return out

    cls.forward = forward
    cls._h3_tp2_amd_swiglu = True
    _state["level"] = level
    return True


def install(level: int = 1, tr=None, check: bool = True) -> bool:  # noqa: ANN001
    """Wrap ``MiniMaxH3MLP.forward`` of the transformer module ``tr`` (default: vLLM-Omni's MiniMax H3) and register
    the stash hook.  With ``check`` kernel 3's install check decides between the fused GEMM and the fp32 stash."""
    if level not in (1, 2):
        raise ValueError(f"unknown SwiGLU level {level!r}")
    if tr is None:
        from vllm_omni.diffusion.models.minimax_h3 import minimax_h3_transformer as tr  # noqa: PLC0415
    try:
        from vllm.lora.layers import BaseLayerWithLoRA  # noqa: PLC0415
        lora = (BaseLayerWithLoRA,)
    except ImportError:
        lora = ()
    if check:
        probe_gemm_swiglu("cuda")
    else:
        _state["gemm_swiglu"] = True
    if not _install_on(tr.MiniMaxH3MLP, level=level, lora_layer_type=lora):
        return False
    fp8_gemm.set_stash_hook(_stash_hook)
    logger.warning("h3_tp2_amd: fused FP8 gate/up GEMM + SwiGLU for the MLP ON, level %d (%s)", level,
                   "kernel 3" if _state["gemm_swiglu"] else "fp32 stash + standalone pass")
    return True


def stats() -> dict:
    return dict(_stats)
