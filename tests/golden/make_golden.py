"""Writes the golden fixtures of tests/golden/ (run once: ``python tests/golden/make_golden.py``).

The expected outputs come from torch's and numpy's own CPU routines applied in the order the reference's eager CPU
mirrors apply them -- not from the oracle under test:

* quant.npz        ``quant_torch`` (h3_tp2/fp8_quant_fuse.py:302-307): amax = |x|.max(-1) in fp32,
                   scale = clamp(amax / 448, min=1/(448*512)), q = (x.float() * scale.reciprocal()).clamp(+-448) cast by
                   torch to float8_e4m3fn.  Rows: seeded log-normal activations with x40 outlier columns, an all-zero
                   row (the reference's tests/test_fp8_quant_fuse.py:367-377), a row of bf16 maxima and subnormals.
* amax_sweep.npz   the same formula with every positive finite bf16 as a row maximum (bits 0x0001..0x7f7f; the
                   reference's sweep in tests/test_fp8_quant_fuse_gpu.py:121-134, at K = 8).
* epilogue.npz     ``scale_bias_cast_torch`` / ``epilogue_torch`` (h3_tp2/fp8_gemm.py:120-126, :174-185):
                   t = sb * acc, y = sa * t in fp32, then torch's cast to bf16 and to fp16; with a bias the exact value
                   sa * t + bias (Python fractions) rounded once to fp32, then cast (one fma).
* swiglu.npz       ``swiglu_epilogue_torch`` (h3_tp2/fp8_swiglu.py:203-212) on the directed values of
                   tests/test_fp8_swiglu.py:31-45 plus seeded rows, with the exp of the silu taken in float64 by numpy
                   and rounded once to fp32 (the correctly rounded exp); ``silu_torch_exp`` is the 65536-entry silu
                   table with torch's own fp32 exp instead (the reference's CPU mirror as it runs).
"""
from __future__ import annotations

import os
from fractions import Fraction

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
FP8_MAX = 448.0
MIN_SCALE = 1.0 / (448.0 * 512.0)
E4M3 = torch.float8_e4m3fn


def quant_torch(h: torch.Tensor):
    x_max = h.abs().max(dim=-1)[0].unsqueeze(-1).to(torch.float32)
    scale = (x_max / FP8_MAX).clamp(min=MIN_SCALE)
    out = (h.to(torch.float32) * scale.reciprocal()).clamp(-FP8_MAX, FP8_MAX).to(E4M3)
    return out, scale


def bits16(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def f32_round(fr: Fraction) -> np.float32:
    """Correctly rounded (nearest even) fp32 of an exact rational, normal range only."""
    if fr == 0:
        return np.float32(0.0)
    sign = -1 if fr < 0 else 1
    fr = abs(fr)
    e = fr.numerator.bit_length() - fr.denominator.bit_length()
    if Fraction(2) ** e > fr:
        e -= 1
    scaled = fr / Fraction(2) ** (e - 23)            # in [2^23, 2^24)
    n = scaled.numerator // scaled.denominator
    rem = scaled - n
    if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and n % 2):
        n += 1
    return np.float32(sign * float(n) * 2.0 ** (e - 23))


def make_quant():
    g = torch.Generator().manual_seed(11)
    M, K = 64, 512
    x = torch.randn(M, K, generator=g) * torch.exp(torch.randn(M, 1, generator=g) * 2.0)
    cols = torch.randperm(K, generator=g)[:4]
    x[:, cols] *= 40.0
    x[3] = 0.0                                                     # all-zero row: MIN_SCALE
    x[5] = torch.linspace(-1.0, 1.0, K) * 3.3895313892515355e38    # bf16 maxima
    x[7] = torch.randn(K, generator=g) * 1e-39                      # subnormal row
    x[9, :8] = torch.tensor([448.0, -448.0, 0.5, -0.5, 1e-30, -1e-30, 0.0, -0.0])
    xb = x.to(torch.bfloat16)
    q, s = quant_torch(xb)
    np.savez_compressed(os.path.join(HERE, "quant.npz"), x=bits16(xb), q=q.view(torch.uint8).numpy(),
                        scale=s.numpy().reshape(-1))


def make_amax_sweep():
    g = torch.Generator().manual_seed(12)
    amax_bits = np.arange(0x0001, 0x7F80, dtype=np.uint16)          # every positive finite bf16
    amax = torch.from_numpy(amax_bits.astype(np.int16)).view(torch.bfloat16).float()
    frac = torch.rand(len(amax_bits), 6, generator=g) * 2.0 - 1.0
    x = torch.cat([amax[:, None], -amax[:, None], amax[:, None] * frac], 1).to(torch.bfloat16)
    q, s = quant_torch(x)
    np.savez_compressed(os.path.join(HERE, "amax_sweep.npz"), x=bits16(x), q=q.view(torch.uint8).numpy(),
                        scale=s.numpy().reshape(-1))


def make_epilogue():
    g = torch.Generator().manual_seed(13)
    M, N = 32, 64
    acc = torch.randn(M, N, generator=g) * 1000.0
    acc[0, 0] = 1.0000001192092896                                  # 1 + 2^-23: the order-sensitive case
    acc[1, :4] = torch.tensor([0.0, -0.0, 3.0e38, -3.0e38])
    sa = torch.exp(torch.empty(M).uniform_(-9.0, -2.0, generator=g))
    sb = torch.exp(torch.empty(N).uniform_(-9.5, -7.5, generator=g))
    sa[0], sb[0] = 3.0, 0.1
    y32 = (sb.view(1, -1) * acc) * sa.view(-1, 1)
    bias = (torch.randn(N, generator=g) * 0.05).to(torch.bfloat16)
    t = (sb.view(1, -1) * acc).numpy()
    sa_n, bias_n = sa.numpy(), bias.float().numpy()
    yb = np.empty((M, N), np.float32)
    for m in range(M):
        for n in range(N):
            yb[m, n] = f32_round(Fraction(float(sa_n[m])) * Fraction(float(t[m, n])) + Fraction(float(bias_n[n])))
    np.savez_compressed(os.path.join(HERE, "epilogue.npz"), acc=acc.numpy(), sa=sa.numpy(), sb=sb.numpy(),
                        bias=bits16(bias), y_bf16=bits16(y32.to(torch.bfloat16)),
                        y_fp16=bits16(y32.to(torch.float16)),
                        y_bias_bf16=bits16(torch.from_numpy(yb).to(torch.bfloat16)))


def silu_rows(g32: torch.Tensor, exp_fn) -> torch.Tensor:
    s = (g32 / (1.0 + exp_fn(-g32))).to(torch.bfloat16).float()
    return s


def exp_cr(x: torch.Tensor) -> torch.Tensor:
    return torch.from_numpy(np.exp(x.double().numpy()).astype(np.float32))


def make_swiglu():
    g = torch.Generator().manual_seed(14)
    width = 2 * 1500
    vals = torch.tensor([0.0, -0.0, 1e-40, -1e-40, 1.0, -1.0, 88.0, -88.0, 1e4, -1e4, 0.5000001, 1.9999999,
                         float("inf"), -float("inf"), float("nan")])
    x32 = vals.repeat(1, width // vals.numel() + 1)[:, :width].clone()
    x32 = torch.cat([x32, torch.randn(7, width, generator=g) * 100, torch.randn(4, width, generator=g) * 3])
    M = x32.shape[0]
    sa = torch.exp(torch.empty(M).uniform_(-1.0, 1.0, generator=g))
    sb = torch.exp(torch.empty(width).uniform_(-1.0, 1.0, generator=g))
    sa[0], sb[:] = 1.0, torch.where(torch.arange(width) < 100, torch.ones(width), sb)
    hb = ((sb.view(1, -1) * x32) * sa.view(-1, 1)).to(torch.bfloat16).float()
    half = width // 2
    gt, u = hb[:, :half], hb[:, half:]
    u = torch.where(u == 0, u.abs(), u)
    h = (silu_rows(gt, exp_cr) * u).to(torch.bfloat16)
    allg = torch.from_numpy(np.arange(65536, dtype=np.uint32).astype(np.uint16).view(np.int16)).view(
        torch.bfloat16).float()
    silu_torch = silu_rows(allg, torch.exp).to(torch.bfloat16)
    np.savez_compressed(os.path.join(HERE, "swiglu.npz"), x32=x32.numpy(), sa=sa.numpy(), sb=sb.numpy(),
                        h=bits16(h), silu_torch_exp=bits16(silu_torch))


if __name__ == "__main__":
    make_quant()
    make_amax_sweep()
    make_epilogue()
    make_swiglu()
    for f in sorted(os.listdir(HERE)):
        if f.endswith(".npz"):
            print(f, os.path.getsize(os.path.join(HERE, f)), "bytes")
