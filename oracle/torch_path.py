"""The reference's torch CPU path of the online-FP8 linear set, restated in torch CPU ops -- TEST INFRASTRUCTURE ONLY.

Only ``bench.py``'s ``cpu_baseline`` leg (which times it on the host's cores) and ``tests/`` (which pin it against the C
oracle) may import this module; the product path never calls it.  Each function follows the reference's eager torch
mirror named beside it (paths relative to the reference checkout):

* ``quant``         h3_tp2/fp8_quant_fuse.py:302-307 (``quant_torch``): amax over the bf16 row, scale =
                    clamp(amax / 448, min=MIN_SCALE), q = clamp(x * reciprocal(scale), +-448) cast to e4m3fn
* ``product``       h3_tp2/fp8_consumers.py:518-523 (``_product_fp32`` on the CPU): ``a.float() @ w.float().t()``
* ``epilogue``      h3_tp2/fp8_gemm.py:174-185 (``epilogue_torch`` without a bias): (sb * acc) * sa, one rounding
* ``swiglu``        h3_tp2/fp8_swiglu.py:203-212 (``swiglu_epilogue_torch``): gate / up through the epilogue, -0 up
                    -> +0, s = bf16(g / (1 + exp(-g))), h = bf16(s * u)
* ``chain_step``    the four linears of a DiT block as the benchmark's block-chain workload runs them on the GPU
                    (QKV; out-projection + the next input's quant; gate/up + SwiGLU + requant; down + the next block's
                    quant), each as quant -> product -> epilogue

``tests/test_oracle.py`` checks that ``quant``, ``epilogue`` and ``swiglu`` give the C oracle's bits on the same inputs.
"""
from __future__ import annotations

import torch

FP8_MAX = 448.0
MIN_SCALE = 1.0 / (FP8_MAX * 512.0)
E4M3 = torch.float8_e4m3fn


def quant(h: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """bf16 [M, K] -> (e4m3fn [M, K], fp32 scale [M, 1])."""
    x_max = h.abs().max(dim=-1)[0].unsqueeze(-1).to(torch.float32)
    scale = (x_max / FP8_MAX).clamp(min=MIN_SCALE)
    return (h.to(torch.float32) * scale.reciprocal()).clamp(-FP8_MAX, FP8_MAX).to(E4M3), scale


def product(a: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
    """fp32 [M, N] = a [M, K] (e4m3fn) times w [N, K] (e4m3fn) transposed, in fp32."""
    return a.float() @ w.float().t()


def epilogue(acc: torch.Tensor, sa: torch.Tensor, sb: torch.Tensor) -> torch.Tensor:
    """bf16 (sb[n] * acc[m, n]) * sa[m]."""
    return (sa.view(-1, 1).float() * (sb.view(1, -1).float() * acc)).to(torch.bfloat16)


def swiglu(acc: torch.Tensor, sa: torch.Tensor, sb: torch.Tensor) -> torch.Tensor:
    """fp32 [M, 2F] accumulator of the merged [gate | up] GEMM -> bf16 h [M, F]."""
    h = epilogue(acc, sa, sb).float()
    half = h.shape[1] // 2
    g, u = h[:, :half], h[:, half:]
    u = torch.where(u == 0, u.abs(), u)
    s = (g / (1.0 + torch.exp(-g))).to(torch.bfloat16).float()
    return (s * u).to(torch.bfloat16)


def linear(x: torch.Tensor, w: torch.Tensor, sw: torch.Tensor) -> torch.Tensor:
    """One online-FP8 linear: per-token quant of x, fp32 product with the quantised weight, epilogue to bf16."""
    q, s = quant(x)
    return epilogue(product(q, w), s, sw)


def chain_step(x: torch.Tensor, x_attn: torch.Tensor, weights: dict) -> tuple[torch.Tensor, torch.Tensor]:
    """One DiT block's linear set on bf16 token rows: ``weights`` maps qkv / out / gate_up / down to (w e4m3fn [N, K],
    sw fp32 [N]).  ``x_attn`` stands in for the attention output that feeds the out-projection.  Returns the QKV output
    and the next block's quantised input (q, as the GPU chain's last stage leaves it)."""
    y_qkv = linear(x, *weights["qkv"])
    y_out = linear(x_attn, *weights["out"])
    qg, sg = quant(y_out)
    h = swiglu(product(qg, weights["gate_up"][0]), sg, weights["gate_up"][1])
    qh, sh = quant(h)
    y_d = epilogue(product(qh, weights["down"][0]), sh, weights["down"][1])
    return y_qkv, quant(y_d)[0]
