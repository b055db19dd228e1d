"""Kernel 3 (SwiGLU epilogue + per-token requant) and its standalone forms against the oracle, bit for bit.

Follows the reference's tests/test_fp8_swiglu.py:17-45, :91-105 (random and directed gate values: +-0, subnormals,
+-88, +-1e4, midpoints, +-inf, NaN, a masked tail) and tests/test_fp8_quant_fuse_gpu.py:93-103 (silu_and_mul + quant
with directed gate/up pairs).  The fused GEMM + SwiGLU is exact on integer-valued operands (exact accumulators).
"""
import numpy as np
import pytest
import torch

from _util import abs_products, assert_quant_equal, bits16, bits8, check_close_swiglu, f32, int_operands, serving_like
from oracle import oracle as O

pytestmark = pytest.mark.gpu


def _nan_aware_equal(out_bits: np.ndarray, ref_bits: np.ndarray):
    nan_ref = (ref_bits & 0x7FFF) > 0x7F80
    nan_out = (out_bits & 0x7FFF) > 0x7F80
    assert np.array_equal(nan_out, nan_ref), "NaN positions differ"
    bad = (out_bits != ref_bits) & ~nan_ref
    assert not bad.any(), f"{int(bad.sum())} bf16 values differ, first at {np.argwhere(bad)[:5].tolist()}"


def test_silu_table_exhaustive(cuda):
    from h3_tp2_amd import ops
    tab = ops.silu_table(cuda).cpu().numpy().view(np.uint16)
    _nan_aware_equal(tab, O.silu_table())


@pytest.mark.parametrize("bias", [False, True])
@pytest.mark.parametrize("M,width", [(64, 256), (300, 28672), (33, 16384)])
def test_scale_swiglu_random(cuda, M, width, bias):
    from h3_tp2_amd import ops
    g = torch.Generator().manual_seed(M + width)
    x32 = torch.randn(M, width, generator=g) * 3000          # gate values up to ~ +-15 after the scales
    sa = torch.rand(M, generator=g) * 0.01 + 0.001
    sb = torch.rand(width, generator=g) * 0.01 + 0.001
    bb = (torch.randn(width, generator=g) * 0.1).to(torch.bfloat16) if bias else None
    h = ops.scale_swiglu(x32.to(cuda), sa.to(cuda), sb.to(cuda), bb.to(cuda) if bias else None)
    q, s = ops.scale_swiglu_quant(x32.to(cuda), sa.to(cuda), sb.to(cuda), bb.to(cuda) if bias else None)
    torch.cuda.synchronize()
    bbits = bits16(bb) if bias else None
    _nan_aware_equal(bits16(h), O.scale_swiglu(x32.numpy(), sa.numpy(), sb.numpy(), bbits))
    assert_quant_equal(q, s, *O.scale_swiglu_quant(x32.numpy(), sa.numpy(), sb.numpy(), bbits))


def test_scale_swiglu_directed_values(cuda):
    from h3_tp2_amd import ops
    width = 2 * 1500
    vals = torch.tensor([0.0, -0.0, 1e-40, -1e-40, 1.0, -1.0, 88.0, -88.0, 1e4, -1e4, 0.5000001, 1.9999999,
                         float("inf"), -float("inf"), float("nan")])
    x32 = vals.repeat(1, width // vals.numel() + 1)[:, :width].clone()
    x32 = torch.cat([x32, torch.randn(7, width, generator=torch.Generator().manual_seed(9)) * 100])
    sa = torch.ones(x32.shape[0])
    sb = torch.ones(width)
    h = ops.scale_swiglu(x32.to(cuda), sa.to(cuda), sb.to(cuda))
    torch.cuda.synchronize()
    _nan_aware_equal(bits16(h), O.scale_swiglu(x32.numpy(), sa.numpy(), sb.numpy()))


def _swiglu_case(M: int, F: int, pad: int, bias: bool, seed: int):
    """An fp32 product [M, 2F] (rows padded by pad floats) with values that force the full-table lookups: a zero
    gate (row 1), a -0 up (row 2), a NaN gate (row 3, a NaN row maximum) and an inf up (row 4)."""
    g = torch.Generator().manual_seed(seed)
    base = torch.randn(M, 2 * F + pad, generator=g) * 3000
    base[1, 3] = 0.0
    base[2, F + 5] = -0.0
    base[3, 7] = float("nan")
    base[4, F + 1] = float("inf")
    sa = torch.rand(M, generator=g) * 0.01 + 0.001
    sb = torch.rand(2 * F, generator=g) * 0.01 + 0.001
    bb = (torch.randn(2 * F, generator=g) * 0.1).to(torch.bfloat16) if bias else None
    return base, sa, sb, bb


# The LDS-table kernels of the fp32 passes, one case per launch shape: 1, 2 and 4 column groups per thread over 4, 8
# and 16 waves (F = 128 ... 16 384) and F past that (the one-workgroup-per-row kernel); several rows per workgroup
# (M = 5001), odd M (a row pair with one row), padded rows.
@pytest.mark.parametrize("M,F,pad", [(5001, 128, 0), (2501, 1000, 8), (700, 2048, 0), (300, 4000, 0), (101, 8184, 4),
                                     (40, 12000, 0), (23, 16384, 0), (9, 16388, 0)])
@pytest.mark.parametrize("bias", [False, True])
def test_scale_swiglu_lds_forms(cuda, M, F, pad, bias):
    from h3_tp2_amd import ops
    base, sa, sb, bb = _swiglu_case(M, F, pad, bias, seed=M * 3 + F)
    xd = base.to(cuda)[:, :2 * F]
    bd = bb.to(cuda) if bias else None
    h = ops.scale_swiglu(xd, sa.to(cuda), sb.to(cuda), bd)
    q, s = ops.scale_swiglu_quant(xd, sa.to(cuda), sb.to(cuda), bd)
    torch.cuda.synchronize()
    x = base[:, :2 * F].contiguous().numpy()
    bbits = bits16(bb) if bias else None
    _nan_aware_equal(bits16(h), O.scale_swiglu(x, sa.numpy(), sb.numpy(), bbits))
    assert_quant_equal(q, s, *O.scale_swiglu_quant(x, sa.numpy(), sb.numpy(), bbits))


# Column scales that are not one contiguous vector take the element-wise and one-workgroup-per-row kernels.
@pytest.mark.parametrize("sb_kind", ["strided", "scalar"])
def test_scale_swiglu_noncontiguous_scales(cuda, sb_kind):
    from h3_tp2_amd import ops
    M, F = 37, 2000
    base, sa, sb, bb = _swiglu_case(M, F, 0, True, seed=5)
    if sb_kind == "strided":
        sbd = torch.stack([sb, sb * 2], dim=1).reshape(-1).to(cuda)[::2]      # stride 2
    else:
        sb = torch.full((2 * F,), 0.004)
        sbd = torch.tensor([0.004]).to(cuda)
    h = ops.scale_swiglu(base.to(cuda), sa.to(cuda), sbd, bb.to(cuda))
    q, s = ops.scale_swiglu_quant(base.to(cuda), sa.to(cuda), sbd, bb.to(cuda))
    torch.cuda.synchronize()
    _nan_aware_equal(bits16(h), O.scale_swiglu(base.numpy(), sa.numpy(), sb.numpy(), bits16(bb)))
    assert_quant_equal(q, s, *O.scale_swiglu_quant(base.numpy(), sa.numpy(), sb.numpy(), bits16(bb)))


def test_swiglu_passes_captured_in_a_graph_replay_bitwise(cuda):
    """The fp32 SwiGLU passes (the LDS-table kernels, with a bias) and the 16-wave bf16 pass captured in one HIP graph
    (torch.cuda.graph) after an eager call: three replays, each after every output was overwritten and the same work
    ran eagerly, with a synchronisation in between, equal the eager results byte for byte."""
    from h3_tp2_amd import ops
    base, sa, sb, bb = _swiglu_case(300, 4000, 0, True, seed=21)
    x, sa_d, sb_d, bb_d = base.to(cuda), sa.to(cuda), sb.to(cuda), bb.to(cuda)
    xb = (torch.randn(40, 2 * 12008, generator=torch.Generator().manual_seed(22)) * 4).to(torch.bfloat16).to(cuda)

    def run():
        return (ops.scale_swiglu(x, sa_d, sb_d, bb_d), *ops.scale_swiglu_quant(x, sa_d, sb_d, bb_d),
                *ops.silu_mul_quant(xb))

    ref = [t.clone() for t in run()]
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        outs = run()
    for rep in range(3):
        for t in outs:
            t.view(torch.uint8).fill_(0x7F)
        run()                                               # eager work between the replays
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for t, r in zip(outs, ref):
            assert torch.equal(t.view(torch.uint8), r.view(torch.uint8)), f"replay {rep}"
    del g


@pytest.mark.parametrize("M,F", [(1, 14336), (200, 14336), (64, 8192), (5, 40000)])
def test_silu_mul_quant(cuda, M, F):
    from h3_tp2_amd import ops
    g = torch.Generator().manual_seed(M + 3)
    h = (torch.randn(M, 2 * F, generator=g) * 4).to(torch.bfloat16)
    h[:, :7] = torch.tensor([0.0, -0.0, 1e-38, -88.0, 88.0, 3.0, -3.0]).to(torch.bfloat16)
    h[:, F:F + 7] = torch.tensor([-0.0, 0.0, -0.0, 1.0, -1.0, -0.0, 0.0]).to(torch.bfloat16)
    q, s = ops.silu_mul_quant(h.to(cuda))
    torch.cuda.synchronize()
    hh = O.swiglu_bf16(bits16(h))
    assert_quant_equal(q, s, *O.quant_rows(hh))


# Shapes of the persistent LDS-table forms (F % 8 == 0; one wave per row up to F = 8192, 16 waves per row up to
# 16 384): ragged 16-byte chunk counts per lane (F = 1000, 520, 8184, 9000, 12 008), one workgroup with idle waves
# (M = 3), several rows per wave or workgroup (M = 4500 over at most 2048 waves, M = 2100 over 256 workgroups), and
# strided inputs (a row stride past 2F).
@pytest.mark.parametrize("M,F,pad", [(3, 1000, 0), (4500, 520, 0), (2600, 8192, 0), (77, 8184, 0), (300, 4096, 24),
                                     (2100, 9000, 0), (37, 16384, 8), (3, 12008, 0)])
def test_silu_mul_quant_persistent_form(cuda, M, F, pad):
    from h3_tp2_amd import ops
    g = torch.Generator().manual_seed(M * 7 + F)
    base = (torch.randn(M, 2 * F + pad, generator=g) * 4).to(torch.bfloat16)
    base[:, :7] = torch.tensor([0.0, -0.0, 1e-38, -88.0, 88.0, 3.0, -3.0]).to(torch.bfloat16)
    base[:, F:F + 7] = torch.tensor([-0.0, 0.0, -0.0, 1.0, -1.0, -0.0, 0.0]).to(torch.bfloat16)
    if M > 2:
        base[1, 5] = float("nan")            # NaN gate: NaN h, NaN row maximum
        base[2, F + 3] = float("inf")        # inf up: inf h in row 2
    x = base[:, :2 * F]
    q, s = ops.silu_mul_quant(base.to(cuda)[:, :2 * F])
    torch.cuda.synchronize()
    hh = O.swiglu_bf16(bits16(x.contiguous()))
    assert_quant_equal(q, s, *O.quant_rows(hh))


@pytest.mark.parametrize("M,F,K", [(200, 320, 512), (333, 1024, 1024), (257, 4096, 3072), (64, 8192, 256),
                                   (1, 128, 64)])
@pytest.mark.parametrize("bias", [False, True])
def test_gemm_swiglu_integer_exact(cuda, M, F, K, bias):
    from h3_tp2_amd import ops
    a, w, sa, sb = int_operands(M, 2 * F, K, seed=M + F + K, device=cuda)
    # scales chosen so the gate values span the interesting part of silu (|g| up to ~10)
    sb = sb * 40.0
    bb = (torch.randn(2 * F, generator=torch.Generator().manual_seed(1)) * 0.5).to(torch.bfloat16).to(cuda) \
        if bias else None
    acc = O.matmul_f32(bits8(a), bits8(w))
    bbits = bits16(bb) if bias else None
    h_ref = O.scale_swiglu(acc, f32(sa), f32(sb), bbits)
    amax = torch.full((M,), 5.0, device=cuda)
    h = ops.gemm_swiglu(a, w, sa, sb, bb, row_amax=amax)
    q, s = ops.gemm_swiglu_quant(a, w, sa, sb, bb)
    torch.cuda.synchronize()
    _nan_aware_equal(bits16(h), h_ref)
    assert torch.equal(amax, h.float().abs().amax(dim=1))
    assert_quant_equal(q, s, *O.scale_swiglu_quant(acc, f32(sa), f32(sb), bbits))


@pytest.mark.parametrize("M", [200, 1000])
def test_gemm_swiglu_random_within_tolerance(cuda, M):
    """Serving-like fc1 operands: the fused kernel against the oracle's SwiGLU of the exact product, within the bound
    propagated from one bf16 ulp plus the MFMA accumulation error on g and u (_util.check_close_swiglu), and equal to
    the oracle's SwiGLU of the kernel's own fp32 accumulator bit for bit (the epilogue itself is exact)."""
    from h3_tp2_amd import ops
    F, K = 4096, 5376
    a, w, sa, sb = serving_like(M, 2 * F, K, seed=M + 17, device=cuda)
    h = ops.gemm_swiglu(a, w, sa, sb)
    acc_gpu = ops.gemm(a, w, sa, sb, torch.float32)
    torch.cuda.synchronize()
    assert np.array_equal(bits16(h), O.scale_swiglu(f32(acc_gpu), f32(sa), f32(sb)))
    A = O.e4m3_to_f32(bits8(a)).astype(np.float64)
    W = O.e4m3_to_f32(bits8(w)).astype(np.float64)
    check_close_swiglu(h, A @ W.T, sa, sb, abs_products(a, w))


def _gate_sweep(gate_bits: np.ndarray, M: int, device):
    """Kernel 3 operands whose accumulator is exactly 1 at every (m, n) (a[:, 0] = w[:, 0] = 1, zeros elsewhere), with
    scale_a = 1, the gate column f's weight scale = the bf16 value gate_bits[f] (exact in fp32) and every up column's
    weight scale 1: the gate of column f is that bf16 value and h = bf16(silu(g) * 1)."""
    F, K = len(gate_bits), 128
    a = torch.zeros(M, K)
    a[:, 0] = 1
    w = torch.zeros(2 * F, K)
    w[:, 0] = 1
    gates = torch.from_numpy(gate_bits.astype(np.uint16).view(np.int16)).view(torch.bfloat16).float()
    sb = torch.cat([gates, torch.ones(F)])
    return (a.to(torch.float8_e4m3fn).to(device), w.to(torch.float8_e4m3fn).to(device), torch.ones(M, device=device),
            sb.to(device), np.ones((M, 2 * F), np.float32), np.ones(M, np.float32), sb.numpy())


def test_gemm_swiglu_every_gate_bit_pattern(cuda):
    """All 65536 bf16 gate values through kernel 3's SiLU lookup (zeros, subnormals, the compact LDS table's range and
    both its edges, huge values, infinities, NaNs): passes whose gates all lie in the compact range take the LDS
    table, the others the full table; either way the oracle's entry."""
    from h3_tp2_amd import ops
    a, w, sa, sb, acc, sa_np, sb_np = _gate_sweep(np.arange(65536), 64, cuda)
    h = ops.gemm_swiglu(a, w, sa, sb)
    torch.cuda.synchronize()
    _nan_aware_equal(bits16(h), O.scale_swiglu(acc, sa_np, sb_np))


def test_gemm_swiglu_compact_table_on_the_fast_path(cuda):
    """Only gates inside the compact table's range (2.6e-9 <= |g| <= 88.5, both signs), laid out in its key order and
    128 columns per weight tile, so every pass of every wave stays on the LDS path and every entry of the table --
    first and last included -- is read from LDS.  Also the rows' maxima."""
    from h3_tp2_amd import ops
    r0, length = 0x6264, 8960                  # the compact table's first rotated key and its length
    keys = np.arange(r0, r0 + length)
    bits = ((keys & 1) << 15) | (keys >> 1)    # rotated key -> bf16 bits
    mag = np.abs(O.bf16_to_f32(bits.astype(np.uint16)))
    assert mag.min() > 2.5e-9 and mag.max() < 89 and np.isfinite(mag).all()
    a, w, sa, sb, acc, sa_np, sb_np = _gate_sweep(bits, 96, cuda)
    amax = torch.zeros(96, device=cuda)
    h = ops.gemm_swiglu(a, w, sa, sb, row_amax=amax)
    torch.cuda.synchronize()
    ref = O.scale_swiglu(acc, sa_np, sb_np)
    assert np.array_equal(bits16(h), ref)
    assert torch.equal(amax, h.float().abs().amax(dim=1))


def test_ffn_full_size_swiglu_requant_is_the_oracle_of_the_accumulator(cuda):
    """The 1344x768 5 s fused FFN at its full size (M = 31248, gate/up 3072 -> 2 x 8192): the fused gate/up GEMM +
    SwiGLU + requant equals, bit for bit, the oracle's SwiGLU and quant applied to the kernel's own fp32 accumulator
    (the raw-accumulator mode of the same GEMM), and the bf16 row of the SwiGLU form equals the oracle's too."""
    from h3_tp2_amd import ops, synthetic
    c = synthetic.CONFIGS["c3_ffn_1344x768_5s"]
    M, K, F = c["M"], c["K"], c["F"]
    x = synthetic.activations(M, K, seed=0, n_out=c["n_out"]).to(cuda)
    a, sa = ops.quant_rows(x)
    del x
    w, sw = ops.quant_rows(synthetic.weight(2 * F, K, seed=2).to(cuda))
    sa, sw = sa.view(-1), sw.view(-1)
    q, s = ops.gemm_swiglu_quant(a, w, sa, sw)
    h = ops.gemm_swiglu(a, w, sa, sw)
    acc = ops.gemm(a, w, sa, sw, torch.float32)
    torch.cuda.synchronize()
    acc_np = f32(acc)
    del acc
    h_ref = O.scale_swiglu(acc_np, f32(sa), f32(sw))
    assert np.array_equal(bits16(h), h_ref)
    assert_quant_equal(q, s, *O.quant_rows(h_ref))
