"""Kernels 2 and 3 on the reference's own H3 DiT linears at serving row counts, against the oracle.

The reference's parity shapes are qkv (N, K) = (21504, 5376), out (5376, 7168), fc1 (28672, 5376) = gate | up of
F = 14336, and fc2 (5376, 14336) (tests/test_fp8_cutlass_gpu.py:19), checked at install on 4100-row serving shapes
(h3_tp2/fp8_cutlass.py:211-213); its published timings are at the per-rank M = 42 848 and the model runs M = 18 880
per rank at 5 s (results/20261103-cutlass-sm120/README.md:30-37).  Here:

* integer-valued operands at M = 4100 (exact accumulators in any order): the whole output equals the oracle bit for
  bit, with guard sentinels around it -- kernel 2 on qkv / out / fc2, kernel 3 (SwiGLU, and SwiGLU + requant) on fc1;
* serving-like operands (log-normal rows exp(N(0, 1) 1.5), N(0, 0.02) weights, both quantised per row by kernel 1) at
  M = 4100 and 18 880: a row sample with at least one row in every 256-row tile row (and the ragged last one) against
  the oracle's epilogue of the exact product, within the per-element tolerance of ``_util.check_close_bf16`` /
  ``check_close_swiglu``; kernel 3's requant bit-exact against the oracle's quant of the kernel's own h.

The exact products of the sampled rows are float64 sums of the dequantised e4m3 codes (computed on the GPU), rounded
once to fp32; the oracle applies the epilogue.
"""
import numpy as np
import pytest
import torch

from _util import (ACC_REL, assert_quant_equal, bits16, check_close_bf16, check_close_swiglu, f32, int_operands)
from oracle import oracle as O

pytestmark = pytest.mark.gpu

H3 = {"qkv": (21504, 5376), "out": (5376, 7168), "fc2": (5376, 14336)}
FC1_F, FC1_K = 14336, 5376


def serving_device(M: int, N: int, K: int, seed: int, device):
    """Serving-like operands made on the device: log-normal activation rows and N(0, 0.02) weights (the reference's
    scripts/fp8_epilogue_probe.py:67-89 distributions), each quantised per row by kernel 1 (bit-exact against the
    oracle's quant, tests/test_quant_gpu.py)."""
    from h3_tp2_amd import ops
    g = torch.Generator(device=device).manual_seed(seed)
    x = (torch.randn(M, K, generator=g, device=device)
         * torch.exp(torch.randn(M, 1, generator=g, device=device) * 1.5)).to(torch.bfloat16)
    w = (torch.randn(N, K, generator=g, device=device) * 0.02).to(torch.bfloat16)
    a, sa = ops.quant_rows(x)
    wq, sw = ops.quant_rows(w)
    del x, w
    return a, wq, sa.view(-1), sw.view(-1)


def sample_rows(M: int, seed: int) -> np.ndarray:
    """Row 0, the last row, one random row in every 256-row tile row and the first row of the ragged last one."""
    rng = np.random.default_rng(seed)
    rows = {0, M - 1, (M // 256) * 256 if M % 256 else M - 256}
    for p in range((M + 255) // 256):
        rows.add(min(M - 1, p * 256 + int(rng.integers(256))))
    return np.array(sorted(r for r in rows if 0 <= r < M))


def exact_rows(a: torch.Tensor, w: torch.Tensor, rows: np.ndarray):
    """(fp32 exact product [R, N], float64 sum_k |a w| [R, N]) of the sampled rows, as numpy arrays."""
    idx = torch.from_numpy(rows).to(a.device)
    A = a.view(torch.uint8).index_select(0, idx).view(a.dtype).float().double()
    W = w.float().double()
    acc = torch.mm(A, W.t()).float().cpu().numpy()
    absum = torch.mm(A.abs(), W.abs().t()).cpu().numpy()
    return acc, absum


def guarded(M: int, N: int, device):
    """An [M, N] bf16 view inside a buffer with sentinel guards on both sides."""
    guard = 4096
    buf = torch.full((M * N + 2 * guard,), float("nan"), device=device, dtype=torch.bfloat16)
    buf[:guard] = 7.0
    buf[-guard:] = 7.0
    return buf, buf[guard:guard + M * N].view(M, N), guard


def exact_int_product(a: torch.Tensor, w: torch.Tensor) -> np.ndarray:
    """The exact fp32 accumulator of integer-valued operands (|acc| <= 8 K < 2^24): float64 on the GPU."""
    return torch.mm(a.float().double(), w.float().double().t()).float().cpu().numpy()


@pytest.mark.parametrize("shape", list(H3))
def test_kernel2_h3_integer_exact_4100(cuda, shape):
    from h3_tp2_amd import ops
    N, K = H3[shape]
    M = 4100
    a, w, sa, sb = int_operands(M, N, K, seed=N + K, device=cuda)
    buf, y, guard = guarded(M, N, cuda)
    ops.gemm(a, w, sa, sb, torch.bfloat16, out=y)
    torch.cuda.synchronize()
    ref = O.epilogue(exact_int_product(a, w), f32(sa).reshape(-1), f32(sb).reshape(-1))
    assert np.array_equal(bits16(y), ref)
    assert bool((buf[:guard] == 7.0).all()) and bool((buf[-guard:] == 7.0).all())


@pytest.mark.parametrize("M", [4100, 18880])
@pytest.mark.parametrize("shape", list(H3))
def test_kernel2_h3_serving_rows(cuda, shape, M):
    from h3_tp2_amd import ops
    N, K = H3[shape]
    a, w, sa, sb = serving_device(M, N, K, seed=M + N, device=cuda)
    y = ops.gemm(a, w, sa, sb)
    torch.cuda.synchronize()
    rows = sample_rows(M, seed=M + K)
    acc, absum = exact_rows(a, w, rows)
    sa_r = f32(sa).reshape(-1)[rows]
    ref = O.epilogue(acc, sa_r, f32(sb).reshape(-1))
    err = np.abs(np.outer(sa_r.astype(np.float64), f32(sb).reshape(-1).astype(np.float64))) * ACC_REL * absum
    check_close_bf16(y[torch.from_numpy(rows).to(cuda)], ref, err)


def test_kernel3_fc1_integer_exact_4100(cuda):
    """Kernel 3 at the reference's fc1 width F = 14 336 (K = 5376): h, the row maxima and the requant (q, scale)
    equal the oracle of the exact accumulator bit for bit, h with guard sentinels."""
    from h3_tp2_amd import ops
    M, F, K = 4100, FC1_F, FC1_K
    a, w, sa, sb = int_operands(M, 2 * F, K, seed=71, device=cuda)
    sb = sb * 40                                         # gates and ups across the SiLU's curved range
    buf, h, guard = guarded(M, F, cuda)
    amax = torch.full((M,), 5.0, device=cuda)
    ops.gemm_swiglu(a, w, sa, sb, row_amax=amax, out=h)
    q, s = ops.gemm_swiglu_quant(a, w, sa, sb)
    torch.cuda.synchronize()
    acc = exact_int_product(a, w)
    sa_n, sb_n = f32(sa).reshape(-1), f32(sb).reshape(-1)
    assert np.array_equal(bits16(h), O.scale_swiglu(acc, sa_n, sb_n))
    assert bool((buf[:guard] == 7.0).all()) and bool((buf[-guard:] == 7.0).all())
    assert torch.equal(amax, h.float().abs().amax(dim=1))
    assert_quant_equal(q, s, *O.scale_swiglu_quant(acc, sa_n, sb_n))


@pytest.mark.parametrize("M", [4100, 18880])
def test_kernel3_fc1_serving_rows(cuda, M):
    """Kernel 3 + requant at fc1 on serving-like operands: sampled rows of h within the propagated SwiGLU tolerance
    of the oracle on the exact product; q and the scales of those rows equal the oracle's quant of the kernel's h."""
    from h3_tp2_amd import ops
    F, K = FC1_F, FC1_K
    a, w, sa, sb = serving_device(M, 2 * F, K, seed=M + 3, device=cuda)
    h = ops.gemm_swiglu(a, w, sa, sb)
    q, s = ops.gemm_swiglu_quant(a, w, sa, sb)
    torch.cuda.synchronize()
    rows = sample_rows(M, seed=M + 5)
    idx = torch.from_numpy(rows).to(cuda)
    acc, absum = exact_rows(a, w, rows)
    check_close_swiglu(h.index_select(0, idx), acc, sa.index_select(0, idx), sb, absum)
    hr = h.index_select(0, idx)
    assert_quant_equal(q.view(torch.uint8).index_select(0, idx), s.index_select(0, idx), *O.quant_rows(bits16(hr)))
