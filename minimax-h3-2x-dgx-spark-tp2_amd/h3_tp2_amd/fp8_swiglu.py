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

from . import _drift, _sites, fp8_gemm, ops

logger = logging.getLogger("h3_tp2_amd.fp8_swiglu")
_notes = _sites.Notes(logger, "h3_tp2_amd fused SwiGLU: ")

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
    """Kernel 3 on fc1's operands (fp8 a [M, K], b [K, 2F] with b.t() contiguous): the MLP's hidden row h, bf16
    [M, F], with the GEMM epilogue and the SwiGLU applied in registers."""
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
    """vLLM's FP8ScaledMMLinearKernel class (looked up once; a caller without vLLM sets ``_state["fc2_kernel_cls"]``)."""
    if _state["fc2_kernel_cls"] is None:
        try:
            from vllm.model_executor.kernels.linear.scaled_mm.ScaledMMLinearKernel import (  # noqa: PLC0415
                FP8ScaledMMLinearKernel)
        except ImportError:
            return None
        _state["fc2_kernel_cls"] = FP8ScaledMMLinearKernel
    return _state["fc2_kernel_cls"]


def _fc2_plain_kernel(fc2):  # noqa: ANN001,ANN202
    """fc2's FP8 scaled-mm kernel when fc2 is the plain layer the model uses (one tensor-parallel rank, no bias added
    by the layer), else None: only then may its input quant be skipped."""
    kcls = _fc2_kernel_cls()
    kernel = getattr(getattr(fc2, "quant_method", None), "fp8_linear", None)
    plain = (getattr(fc2, "tp_size", 1) == 1 and getattr(fc2, "bias", None) is None
             and not getattr(fc2, "skip_bias_add", False))
    return kernel if kcls is not None and isinstance(kernel, kcls) and plain else None


def _fc2_direct(fc2, q: torch.Tensor, scale: torch.Tensor, lead) -> torch.Tensor | None:  # noqa: ANN001
    """fc2 on a pre-quantised input through its own scaled-mm kernel (its ``apply_weights`` would quantise again), or
    None when fc2 is not the plain layer or its weight does not take q's width."""
    kernel = _fc2_plain_kernel(fc2)
    if kernel is None:
        return None
    w, w_s, _, _ = kernel._get_layer_params(fc2)
    if w.shape[0] != q.shape[1]:
        return None
    return kernel.apply_scaled_mm(A=q, B=w, out_dtype=torch.bfloat16, As=scale, Bs=w_s, bias=None,
                                  output_shape=[*lead, w.shape[1]])


class Fc1Stash:
    """What the stash hook kept of fc1: the GEMM's operands (kernel 3 computes the product) or, without kernel 3, its
    fp32 product; the per-token / per-channel scale vectors and the bias.  Either form yields the MLP's hidden row h or
    fc2's quantised input."""
    __slots__ = ("source", "sa", "sb", "bias")

    def __init__(self, source, sa: torch.Tensor, sb: torch.Tensor, bias):  # noqa: ANN001
        self.source, self.sa, self.sb, self.bias = source, sa, sb, bias

    @property
    def fused(self) -> bool:
        return isinstance(self.source, GemmOperands)

    @property
    def width(self) -> int:
        return self.source.shape[1] // 2

    def hidden(self) -> torch.Tensor:
        """bf16 h [M, F]."""
        _stats["fused" if self.fused else "x32"] += 1
        if self.fused:
            return gemm_swiglu(self.source.a, self.source.b, self.sa, self.sb, self.bias)
        return scale_swiglu(self.source, self.sa, self.sb, self.bias)

    def quantised(self):  # noqa: ANN201
        """(fp8 h [M, F], fp32 per-token scale [M, 1])."""
        _stats["fused_quant" if self.fused else "x32"] += 1
        if self.fused:
            return gemm_swiglu_quant(self.source.a, self.source.b, self.sa, self.sb, self.bias)
        return scale_swiglu_quant(self.source, self.sa, self.sb, self.bias)


def _stash_hook(a, b, scale_a, scale_b, out_dtype, bias):  # noqa: ANN001
    """Dispatcher stash hook: on the fc1 GEMM the MLP forward asked for (``_tls.stash_next``), keep an ``Fc1Stash`` in
    ``_tls.stash`` and return an uninitialised bf16 placeholder of the output's shape.  A bf16 output of even width that
    equals the layer's logical width (``_tls.expect_n``, 0 = unknown) qualifies; anything else declines and withdraws
    the request, so the GEMM takes the ordinary path."""
    if not getattr(_tls, "stash_next", False) or out_dtype is not torch.bfloat16:
        return None
    _tls.stash_next = False                            # one request, one GEMM
    M, N = a.shape[0], b.shape[1]
    expect = getattr(_tls, "expect_n", 0)
    if N % 2 or (expect and N != expect):              # padded fc1: not the MLP's merged [gate | up] product
        return None
    sa, sb = fp8_gemm._vec_scales(scale_a, scale_b, M, N)
    source = GemmOperands(a, b) if _state["gemm_swiglu"] else fp8_gemm.product_fp32(a, b)
    _tls.stash = Fc1Stash(source, sa, sb, bias)
    return torch.empty((M, N), device=a.device, dtype=out_dtype)


class _Fc1Capture:
    """Arms the stash request for the fc1 call made inside the ``with`` block and disarms it on the way out, whatever
    happens; ``stash`` is what the hook kept (None: fc1 ran the ordinary way)."""

    def __init__(self, fc1):  # noqa: ANN001
        self.expect = int(getattr(fc1, "output_size_per_partition", 0) or 0)
        self.stash: Fc1Stash | None = None

    def __enter__(self) -> "_Fc1Capture":
        _tls.stash, _tls.expect_n, _tls.stash_next = None, self.expect, True
        return self

    def __exit__(self, *exc) -> None:  # noqa: ANN002
        self.stash = getattr(_tls, "stash", None)
        _tls.stash, _tls.expect_n, _tls.stash_next = None, 0, False


def _install_on(cls, *, level: int, lora_layer_type=()) -> bool:  # noqa: ANN001
    """Wrap ``cls.forward`` (an MLP with ``fc1``, ``act_fn``, ``fc2``); False when already wrapped.

    The wrapped forward runs fc1 under a stash capture.  Nothing captured: the stock activation and fc2.  Captured:
    fc1's placeholder is dropped and the stash yields h for fc2 (level 1), or fc2's quantised input, which fc2's own
    kernel then takes directly (level 2).  An MLP whose fc1 or fc2 carries a LoRA wrapper takes the stock forward (the
    wrapper adds its delta to fc1's returned tensor, which the fused path discards), and so does a level-2 MLP whose fc2
    is not the plain layer (the stock forward recomputes fc1: correct, slower)."""
    if getattr(cls, "_h3_tp2_amd_swiglu", False):
        return False
    stock_forward = cls.forward
    to_fc2_input = level >= 2

    def lora_wrapped(mlp) -> bool:  # noqa: ANN001
        return bool(lora_layer_type) and any(isinstance(layer, lora_layer_type) for layer in (mlp.fc1, mlp.fc2))

    def forward(self, x):  # noqa: ANN001,ANN202
        if lora_wrapped(self):
            return stock_forward(self, x)
        with _Fc1Capture(self.fc1) as cap:
            placeholder, _ = self.fc1(x)
        if cap.stash is None:
            _stats["stock"] += 1
            return self.fc2(self.act_fn(placeholder))[0]
        lead = placeholder.shape[:-1]
        del placeholder                                 # never written
        stash, cap.stash = cap.stash, None
        if to_fc2_input:
            out = _fc2_direct(self.fc2, *stash.quantised(), lead)
            if out is not None:
                _stats["fc2_direct"] += 1
                return out
            _stats["fc2_redo"] += 1
            del stash
            return stock_forward(self, x)
        h = stash.hidden().view(*lead, stash.width)
        del stash                                       # the fp32 product (two-pass form) goes before fc2 allocates
        return self.fc2(h)[0]

    forward.__wrapped__ = stock_forward             # source fingerprints see the upstream forward through it
    forward._h3_tp2_amd_swiglu = True
    cls.forward = forward
    cls._h3_tp2_amd_swiglu = True
    _state["level"] = level
    return True


def install(level: int = 1, tr=None, check: bool = True, *, check_source: bool = True,  # noqa: ANN001
            reviewed: dict | None = None) -> bool:
    """Wrap ``MiniMaxH3MLP.forward`` of the transformer module ``tr`` (default: vLLM-Omni's MiniMax H3) and register
    the stash hook.  With ``check`` kernel 3's install check decides between the fused GEMM and the fp32 stash.  With
    ``check_source`` the MLP forward must fingerprint to the reviewed upstream source (``_drift``): the wrapper relies
    on fc1's output reaching ``act_fn`` and then fc2 and nothing else."""
    if level not in (1, 2):
        raise ValueError(f"unknown SwiGLU level {level!r}")
    if tr is None:
        from vllm_omni.diffusion.models.minimax_h3 import minimax_h3_transformer as tr  # noqa: PLC0415
    if check_source and not _drift.keep_sites("mlp", ("fc1",), tr, _notes, reviewed, modules={}):
        return False
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
