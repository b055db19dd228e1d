"""Helpers shared by the tests: bit views, oracle calls on torch tensors, seeded operand generators."""
from __future__ import annotations

import numpy as np
import torch

from oracle import oracle as O

E4M3 = torch.float8_e4m3fn


def bits16(t: torch.Tensor) -> np.ndarray:
    return t.detach().contiguous().cpu().view(torch.int16).numpy().view(np.uint16)


def bits8(t: torch.Tensor) -> np.ndarray:
    return t.detach().contiguous().cpu().view(torch.uint8).numpy()


def f32(t: torch.Tensor) -> np.ndarray:
    return t.detach().contiguous().cpu().float().numpy()


def oracle_quant(x: torch.Tensor):
    """oracle quant_rows on a bf16 torch tensor: (codes uint8 [M, K], scale fp32 [M])."""
    return O.quant_rows(bits16(x))


def assert_quant_equal(q: torch.Tensor, s: torch.Tensor, q_ref: np.ndarray, s_ref: np.ndarray, nan_rows_ok=True):
    """fp8 bytes and scale bits equal; NaN codes / NaN scales compared by position only."""
    qb, sb = bits8(q), f32(s).reshape(-1)
    assert qb.shape == q_ref.shape, (qb.shape, q_ref.shape)
    nan_q = (q_ref & 0x7F) == 0x7F
    assert np.array_equal((qb & 0x7F) == 0x7F, nan_q), "NaN code positions differ"
    bad = (qb != q_ref) & ~nan_q
    assert not bad.any(), f"{int(bad.sum())} fp8 bytes differ, first at {np.argwhere(bad)[:5].tolist()}"
    nan_s = np.isnan(s_ref)
    assert np.array_equal(np.isnan(sb), nan_s), "NaN scale positions differ"
    sbits, rbits = sb.view(np.uint32), s_ref.astype(np.float32).view(np.uint32)
    bad_s = (sbits != rbits) & ~nan_s
    assert not bad_s.any(), f"{int(bad_s.sum())} scales differ, first rows {np.nonzero(bad_s)[0][:5].tolist()}"


def int_operands(M: int, N: int, K: int, seed: int, device):
    """Integer-valued fp8 operands (a in [-4, 4], w in [-2, 2]): |acc| <= 8K < 2^24, so the fp32 accumulator is exact
    in any summation order (the reference's scripts/fp8_epilogue_probe.py:70-72 and tests/test_fp8_fused_gpu.py)."""
    g = torch.Generator().manual_seed(seed)
    a = torch.randint(-4, 5, (M, K), generator=g).float().to(E4M3)
    w = torch.randint(-2, 3, (N, K), generator=g).float().to(E4M3)
    sa = torch.exp(torch.empty(M).uniform_(-9.0, -2.0, generator=g))
    sb = torch.exp(torch.empty(N).uniform_(-9.5, -7.5, generator=g))
    return a.to(device), w.to(device), sa.to(device), sb.to(device)


def serving_like(M: int, N: int, K: int, seed: int, device):
    """Per-token quantised log-normal activations and per-channel quantised N(0, 0.02) weights
    (the reference's tests/test_fp8_cutlass_gpu.py:_serving_like), quantised by the oracle."""
    g = torch.Generator().manual_seed(seed)
    x = (torch.randn(M, K, generator=g) * torch.exp(torch.randn(M, 1, generator=g) * 1.5)).to(torch.bfloat16)
    w = (torch.randn(N, K, generator=g) * 0.02).to(torch.bfloat16)
    qa, sa = O.quant_rows(bits16(x))
    qw, sw = O.quant_rows(bits16(w))
    a = torch.from_numpy(qa).view(E4M3)
    wq = torch.from_numpy(qw).view(E4M3)
    return a.to(device), wq.to(device), torch.from_numpy(sa).to(device), torch.from_numpy(sw).to(device)


def ref_gemm(a: torch.Tensor, w: torch.Tensor, sa, sb, bias=None, out_fp16=False) -> np.ndarray:
    """oracle: fp32 product of the e4m3 codes (numpy BLAS) + the scaled epilogue -> output bit patterns."""
    acc = O.matmul_f32(bits8(a), bits8(w))
    sa_n = f32(sa).reshape(-1)
    sb_n = f32(sb).reshape(-1)
    b = None if bias is None else bits16(bias)
    return O.epilogue(acc, sa_n, sb_n, b, out_fp16)


def bf16_from_bits(b: np.ndarray) -> np.ndarray:
    return (b.astype(np.uint32) << 16).view(np.float32)


def check_close_bf16(y: torch.Tensor, ref_bits: np.ndarray, min_equal: float = 0.95, row_frac: float = 2.0 ** -10,
                     ulps: float = 1.0):
    """Tolerance for a bf16 GEMM output against the oracle (fp32-accumulated dequantised product, same epilogue).

    The kernel and the oracle sum K in different orders, so their fp32 accumulators differ by a few fp32 ulps and a
    bf16 rounding may flip.  Stated bound, per element:  |y - ref| <= ulp_bf16(ref) + 2^-10 * rms(row of ref)
    (one bf16 ulp, plus an absolute slack for cancellation near zero), and at least ``min_equal`` of the outputs
    bit-equal.  Returns (max |err| / rms, fraction bit-equal).  The whole-tensor form "max |err| <= 2e-2 * rms" is not
    used: one ulp at |y| > 5 rms already exceeds it for bf16 outputs."""
    out = f32(y).astype(np.float64)
    ref = bf16_from_bits(ref_bits).astype(np.float64)
    assert np.isfinite(out).all() and np.isfinite(ref).all()
    mag = np.abs(ref)
    e = np.floor(np.log2(np.where(mag > 0, mag, 1.0)))
    ulp = np.where(mag > 0, np.exp2(e - 7), 0.0)
    row_rms = np.sqrt(np.mean(ref * ref, axis=1, keepdims=True))
    err = np.abs(out - ref)
    bound = ulps * ulp + row_frac * row_rms
    bad = err > bound
    assert not bad.any(), f"{int(bad.sum())} outputs beyond {ulps} ulp + {row_frac} rms_row; worst {np.max(err - bound)}"
    eq = float(np.mean(bits16(y) == ref_bits))
    assert eq >= min_equal, eq
    rms = float(np.sqrt(np.mean(ref * ref)))
    return float(err.max()) / rms, eq
