"""Seeded synthetic DiT activations and weights (no datasets or checkpoints are available offline).

Activations ~ N(0, 1) with ``n_out`` outlier channels (a seeded choice of columns) scaled by 40; weights ~ N(0, 0.02).
Generated on the CPU in fp32 with ``torch.Generator().manual_seed(seed)`` and rounded to bf16, so every run and every
machine produces the same tensors.  The reference's own probe inputs (scripts/fp8_epilogue_probe.py:67-89: per-row
log-normal magnitudes exp(N(0,1) * 1.5)) are available as ``kind="lognormal"``.
"""
from __future__ import annotations

import torch


def activations(M: int, K: int, seed: int, n_out: int = 0, kind: str = "normal") -> torch.Tensor:
    """bf16 [M, K] on the CPU."""
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(M, K, generator=g)
    if kind == "lognormal":
        x *= torch.exp(torch.randn(M, 1, generator=g) * 1.5)
    elif kind != "normal":
        raise ValueError(kind)
    if n_out:
        cols = torch.randperm(K, generator=g)[:n_out]
        x[:, cols] *= 40.0
    return x.to(torch.bfloat16)


def weight(N: int, K: int, seed: int, std: float = 0.02) -> torch.Tensor:
    """bf16 [N, K] on the CPU (an nn.Linear weight: output channels are rows)."""
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(N, K, generator=g) * std).to(torch.bfloat16)


def n_outliers(K: int, frac: float = 0.001) -> int:
    """0.1 % of the channels, at least one."""
    return max(1, round(frac * K))


# The measured workloads (token counts M = latent frames x patches per frame; hidden 3072, QKV 9216, FFN 2 x 8192).
CONFIGS = {
    "c1_single_linear": dict(M=2048, K=3072, N=3072, n_out=8),
    "c2_qkv_960x576_5s": dict(M=16740, K=3072, N=9216, n_out=3),
    "c3_ffn_1344x768_5s": dict(M=31248, K=3072, F=8192, n_out=3),
    "c4_chain_1344x768_15s": dict(M=91728, K=3072, n_out=3),
    "c5_grouped": dict(groups=[(2, 3072, 18432, 3), (512, 4096, 6144, 4), (1600, 1536, 4608, 2),
                               (16740, 3072, 9216, 3)]),
}
