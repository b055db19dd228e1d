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


# Accumulation-error model of the gfx950 FP8 MFMA (v_mfma_f32_32x32x64_f8f6f4): each instruction sums its 64 products
# with well under fp32 precision before adding them to the fp32 accumulator, and the error grows with the dynamic
# range of the products.  Measured max |acc - exact| / sum_k |a_k w_k|: 2^-19.0 on serving-like operands (log-normal
# rows), 2^-14.7 on N(0,1) activations with x40 outlier channels (K = 3072), 2^-15.8 (K = 8192); a sequential fp32 sum
# stays below 2^-25.6.  The tolerances allow ACC_REL = 2^-12 (four times the worst seen); for N(0,1) activations that
# is about 1 % of the output rms.  test_gemm_gpu.py::test_accumulator_error_model pins the bound on the raw fp32
# accumulator.
ACC_REL = 2.0 ** -12


def abs_products(a: torch.Tensor, w: torch.Tensor) -> np.ndarray:
    """sum_k |a[m,k]| |w[n,k]| in float64 (the scale of the accumulation error)."""
    A = np.abs(O.e4m3_to_f32(bits8(a)).astype(np.float64))
    W = np.abs(O.e4m3_to_f32(bits8(w)).astype(np.float64))
    return A @ W.T


def ulp_bf16(x: np.ndarray) -> np.ndarray:
    mag = np.abs(x)
    e = np.floor(np.log2(np.where(mag > 0, mag, 1.0)))
    return np.where(mag > 0, np.exp2(e - 7), 2.0 ** -133)


def check_close_bf16(y: torch.Tensor, ref_bits: np.ndarray, acc_err: np.ndarray, min_equal: float = 0.95):
    """Tolerance for a bf16 GEMM output against the oracle (exact dequantised product, the same epilogue):
    |y - ref| <= ulp_bf16(ref) + acc_err per element, acc_err = |sa sb| * ACC_REL * sum_k |a w| (the MFMA's
    accumulation error carried through the scales), and at least ``min_equal`` of the outputs bit-equal.
    Returns (max |err| / rms, fraction bit-equal).  The whole-tensor form "max |err| <= 2e-2 * rms" is not used: one
    bf16 ulp at |y| > 5 rms already exceeds it."""
    out = f32(y).astype(np.float64)
    ref = bf16_from_bits(ref_bits).astype(np.float64)
    assert np.isfinite(out).all() and np.isfinite(ref).all()
    err = np.abs(out - ref)
    bound = ulp_bf16(ref) + acc_err
    bad = err > bound
    assert not bad.any(), f"{int(bad.sum())} outputs beyond 1 ulp + accumulation error; worst {np.max(err - bound)}"
    eq = float(np.mean(bits16(y) == ref_bits))
    assert eq >= min_equal, eq
    rms = float(np.sqrt(np.mean(ref * ref)))
    return float(err.max()) / rms, eq


def gemm_acc_err(a, w, sa, sb) -> np.ndarray:
    """Per-element bound of the accumulation error after the scales: |sa[m] sb[n]| ACC_REL sum_k |a w|."""
    return np.abs(np.outer(f32(sa).reshape(-1).astype(np.float64), f32(sb).reshape(-1).astype(np.float64))) * \
        ACC_REL * abs_products(a, w)


def check_close_swiglu(h: torch.Tensor, acc_exact: np.ndarray, sa, sb, absum: np.ndarray, min_equal: float = 0.95):
    """Tolerance for the fused gate/up GEMM + SwiGLU.  With the oracle's bf16 gate g, up u and silu s = silu_bf16(g)
    from the exact product, each of g and u may move by one bf16 ulp plus its accumulation error (dg, du), s by up to
    1.1 dg (|silu'| <= 1.1) plus one ulp (ds), and h by |u| ds + |s| du + ds du plus its own rounding."""
    sa_n = f32(sa).reshape(-1).astype(np.float64)
    sb_n = f32(sb).reshape(-1).astype(np.float64)
    F = acc_exact.shape[1] // 2
    g_bits = O.epilogue(acc_exact[:, :F].astype(np.float32), f32(sa).reshape(-1), f32(sb).reshape(-1)[:F])
    u_bits = O.epilogue(acc_exact[:, F:].astype(np.float32), f32(sa).reshape(-1), f32(sb).reshape(-1)[F:])
    g, u = bf16_from_bits(g_bits).astype(np.float64), bf16_from_bits(u_bits).astype(np.float64)
    s = bf16_from_bits(O.silu_table()[g_bits]).astype(np.float64)
    h_ref_bits = O.scale_swiglu(acc_exact.astype(np.float32), f32(sa), f32(sb))
    href = bf16_from_bits(h_ref_bits).astype(np.float64)
    dg = ulp_bf16(g) + np.abs(np.outer(sa_n, sb_n[:F])) * ACC_REL * absum[:, :F]
    du = ulp_bf16(u) + np.abs(np.outer(sa_n, sb_n[F:])) * ACC_REL * absum[:, F:]
    ds = 1.1 * dg + ulp_bf16(s)
    bound = np.abs(u) * ds + np.abs(s) * du + ds * du + ulp_bf16(href)
    out = f32(h).astype(np.float64)
    err = np.abs(out - href)
    bad = err > bound
    assert not bad.any(), f"{int(bad.sum())} SwiGLU outputs beyond the propagated bound; worst {np.max(err - bound)}"
    eq = float(np.mean(bits16(h) == h_ref_bits))
    assert eq >= min_equal, eq
    return eq


def mod_inputs(M: int, H: int, seed: int, B: int = 6, std_scale: float = 1.0):
    """Seeded operands of the RMSNorm + AdaLN producers, shaped like the reference's tests/test_fp8_quant_fuse_gpu.py
    :40-48: rows with log-normal magnitudes, weight ~ 1 + 0.1 N(0, 1), shift / scale / gate as chunk views of one
    [B, 6H] modulation table (row stride 6H), indices in [0, B).  CPU tensors: x, weight, shift, scale, gate, idx."""
    g = torch.Generator().manual_seed(seed)
    mag = torch.exp(torch.randn(M, 1, generator=g) * 1.5)
    x = (torch.randn(M, H, generator=g) * mag).to(torch.bfloat16)
    weight = (1.0 + 0.1 * torch.randn(H, generator=g)).to(torch.bfloat16)
    ada = (torch.randn(B, 6 * H, generator=g) * std_scale).to(torch.bfloat16)
    shift, scale, gate = ada[:, :H], ada[:, H:2 * H], ada[:, 2 * H:3 * H]
    idx = torch.randint(0, B, (M,), generator=g)
    return x, weight, shift, scale, gate, idx


def standin_rms(x, weight, shift, scale, idx, eps):
    """The stock rms_norm_indexed_scale_shift as the reference's CPU stand-in evaluates it (torch CPU ops,
    tests/fake_h3_consumers.py:77-84): bf16 [M, H]."""
    xf = x.float()
    var = (xf * xf).sum(dim=1, keepdim=True) / x.shape[1]
    n = xf * torch.rsqrt(var + eps) * weight.float()
    return (n * (1.0 + scale.index_select(0, idx).float()) + shift.index_select(0, idx).float()).to(torch.bfloat16)


def standin_gate_rms(residual, gate, branch, weight, shift, scale, idx, eps):
    """The stock indexed_gate_rms_norm_scale_shift as the CPU stand-in evaluates it (fake_h3_consumers.py:66-74)."""
    upd = (residual.float() + gate.index_select(0, idx).float() * branch.float()).to(torch.bfloat16)
    return upd, standin_rms(upd, weight, shift, scale, idx, eps)


def standin_qk_norm_rope(x, weight, table, eps):
    """The stock fused_qk_norm_rope half-split kernel as the reference's CPU stand-in evaluates it (torch CPU ops,
    tests/fake_h3_consumers.py:29-48): bf16 [T, H, 128] -> bf16 [T, H, 128]; table [T, 96] (cos | sin)."""
    T, Hh, D = x.shape
    half = table.shape[-1] // 2
    rot = 2 * half
    dims = torch.arange(D)
    xf = x.float()
    w = weight.float()
    inv = torch.rsqrt((xf * xf).sum(dim=-1) / D + eps)
    n = (xf * inv[..., None] * w).to(torch.bfloat16)
    pd = torch.where(dims < half, dims + half, torch.where(dims < rot, dims - half, dims))
    p = (xf[..., pd] * inv[..., None] * w[pd]).to(torch.bfloat16)
    fd = torch.where(dims < half, dims, torch.where(dims < rot, dims - half, torch.zeros_like(dims)))
    cos = table[:, fd].float()[:, None, :]
    sin = table[:, fd + half].float()[:, None, :]
    first = n.float() * cos - p.float() * sin
    second = n.float() * cos + p.float() * sin
    out = torch.where(dims < rot, torch.where(dims < half, first, second), n.float())
    return out.to(x.dtype)


def rope_table(T: int, dtype, seed: int = 3):
    """A rope table [T, 96] = cos | sin of seeded positions times 48 frequencies (the reference's
    tests/test_fp8_consumer_fuse.py:64-67 generator)."""
    g = torch.Generator().manual_seed(seed)
    pos = torch.rand(T, 1, generator=g) * 500 * torch.exp(-torch.arange(48) / 8.0)[None, :]
    return torch.cat((torch.cos(pos), torch.sin(pos)), dim=-1).to(dtype)


# A 128-dim head whose fp32 sum of squares depends on the reduction order: its fp64 sum sits on an fp32 rounding tie
# (large squares that are multiples of the fp32 ulp plus 2^17 squared, half an ulp), and the small squares tip it only
# when they are summed among themselves before they meet the large ones.  With weight ORDER_W at dim ORDER_DIM the
# normalised bf16 output of that dim differs between the kernel's lane order (KERNEL_LANES: lane k adds dims
# 32i + 4k + e in the order i, e = 0 .. 3, then an xor butterfly over 4, 2, 1) and a 32 x 4 one (CONTIG32_LANES), so a
# kernel that reduces in another order fails it.
ORDER_HEAD = {15: 4.0, 31: 131072.0, 41: -4.0, 47: 2.0, 48: 62128128.0, 53: -4.0, 64: 50593792.0, 66: 3.0, 76: -4.0,
              79: 557842432.0, 106: 2.0, 118: -4.0, 126: 4.0}
ORDER_DIM, ORDER_W = 31, 1.40625
KERNEL_LANES = [[32 * i + 4 * k + e for i in range(4) for e in range(4)] for k in range(8)]
CONTIG32_LANES = [[4 * k + e for e in range(4)] for k in range(32)]


def lane_order_sumsq(x, lanes) -> float:
    """fp64 sum of the fp32 squares of a 128-dim head: lane l adds the squares of the dims lanes[l] in that order, then
    an xor butterfly over the lane sums (largest distance first); rounded to fp32."""
    import numpy as np
    p = []
    for dims in lanes:
        s = 0.0
        for d in dims:
            s += float(np.float32(x[d]) * np.float32(x[d]))
        p.append(s)
    d = len(p) // 2
    while d >= 1:
        p = [p[l] + p[l ^ d] for l in range(len(p))]
        d //= 2
    return float(np.float32(p[0]))
