"""Kernel 2 (scaled FP8 GEMM) against the oracle.

* Integer-valued operands make the fp32 accumulator exact in any summation order, so the whole output (epilogue,
  tile map, M/N/K tails, masks) must equal the oracle bit for bit (the reference's tests/test_fp8_cutlass_gpu.py:56-74
  and scripts/fp8_epilogue_probe.py:70-72), with guard sentinels around the output (no write outside [M, N]).
* Random serving-like operands on the reference's DiT shapes and on the measured shapes: within the stated tolerance
  |y - ref| <= ulp_bf16(ref) + |sa sb| 2^-12 sum_k |a w| per element (ref = the exact dequantised product through the
  same epilogue; the second term is the FP8 MFMA's accumulation error, see _util.ACC_REL), and at least 95 % of the
  bf16 outputs bit-equal.
"""
import numpy as np
import pytest
import torch

from _util import (ACC_REL, abs_products, assert_quant_equal, bits8, bits16, check_close_bf16, gemm_acc_err,
                   int_operands, oracle_quant, ref_gemm, serving_like)
from oracle import oracle as O

pytestmark = pytest.mark.gpu

DIT = {"qkv": (21504, 5376), "out": (5376, 7168), "fc1": (28672, 5376), "fc2": (5376, 14336)}
MEASURED = {"c1": (2048, 3072, 3072), "qkv": (16740, 9216, 3072), "down": (31248, 3072, 8192)}


def ref_gemm_exact(a, w, sa, sb):
    """oracle epilogue on the exact (float64-summed, fp32-rounded) product."""
    A = O.e4m3_to_f32(bits8(a)).astype(np.float64)
    W = O.e4m3_to_f32(bits8(w)).astype(np.float64)
    return O.epilogue((A @ W.T).astype(np.float32), sa.cpu().numpy().reshape(-1), sb.cpu().numpy().reshape(-1))


def _gemm(a, w, sa, sb, out_dtype=torch.bfloat16, bias=None):
    from h3_tp2_amd import ops
    y = ops.gemm(a, w, sa, sb, out_dtype, bias)
    torch.cuda.synchronize()
    return y


@pytest.mark.parametrize("M,N,K", [(1, 128, 64), (200, 400, 512), (333, 272, 1024), (129, 5376, 7168),
                                   (8200, 144, 320), (257, 9216, 3072), (512, 256, 128), (300, 1040, 208)])
def test_integer_inputs_exact_with_guards(cuda, M, N, K):
    from h3_tp2_amd import ops
    a, w, sa, sb = int_operands(M, N, K, seed=M + N + K, device=cuda)
    ref = ref_gemm(a, w, sa, sb)
    guard = 4096
    buf = torch.full((M * N + 2 * guard,), float("nan"), device=cuda, dtype=torch.bfloat16)
    buf[:guard] = 7.0
    buf[-guard:] = 7.0
    y = buf[guard:guard + M * N].view(M, N)
    ops.gemm(a, w, sa, sb, torch.bfloat16, out=y)
    torch.cuda.synchronize()
    assert np.array_equal(bits16(y), ref)
    assert bool((buf[:guard] == 7.0).all()) and bool((buf[-guard:] == 7.0).all())


@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("bias", [False, True])
@pytest.mark.parametrize("scalar", ["none", "sa", "sb"])
@pytest.mark.parametrize("N", [528, 400])
def test_integer_inputs_dtypes_bias_scalars(cuda, out_dtype, bias, scalar, N):
    """Output dtypes, bias and scalar scales, exact on integer operands; N = 528 runs as 12 half tiles, N = 400 as
    9 tiles of 128 x 192 (ragged in both M and N)."""
    M, K = 300, 768
    a, w, sa, sb = int_operands(M, N, K, seed=11, device=cuda)
    if scalar == "sa":
        sa = sa[:1].reshape(())
    if scalar == "sb":
        sb = sb[:1].reshape(1, 1)
    bb = (torch.randn(N, generator=torch.Generator().manual_seed(5)) * 0.1).to(out_dtype).to(cuda) if bias else None
    y = _gemm(a, w, sa.reshape(-1, 1) if scalar != "sa" else sa, sb, out_dtype, bb)
    ref = ref_gemm(a, w, sa.reshape(-1).expand(M) if scalar == "sa" else sa,
                   sb.reshape(-1).expand(N) if scalar == "sb" else sb, bb, out_dtype == torch.float16)
    assert y.dtype == out_dtype and np.array_equal(bits16(y), ref)


@pytest.mark.parametrize("M", [200, 1000])
@pytest.mark.parametrize("shape", list(DIT))
def test_dit_shapes_within_tolerance(cuda, shape, M):
    N, K = DIT[shape]
    a, w, sa, sb = serving_like(M, N, K, seed=M * 7 + N, device=cuda)
    y = _gemm(a, w, sa.view(M, 1), sb)
    check_close_bf16(y, ref_gemm_exact(a, w, sa, sb), gemm_acc_err(a, w, sa, sb))


@pytest.mark.parametrize("name", list(MEASURED))
def test_measured_shapes_within_tolerance(cuda, name):
    from h3_tp2_amd import ops, synthetic
    M, N, K = MEASURED[name]
    x = synthetic.activations(M, K, seed=0, n_out=synthetic.n_outliers(K))
    wt = synthetic.weight(N, K, seed=1)
    a, sa = ops.quant_rows(x.to(cuda))
    w, sb = ops.quant_rows(wt.to(cuda))
    y = _gemm(a, w, sa, sb)
    check_close_bf16(y, ref_gemm_exact(a, w, sa, sb), gemm_acc_err(a, w, sa, sb))


@pytest.mark.parametrize("M,N,K", [(777, 3072, 1024), (4100, 4368, 256), (2300, 3600, 256)])
def test_fused_row_amax_and_quant(cuda, M, N, K):
    """The fused next-layer quant: the row maxima and the quant from them equal the plain GEMM's output and kernel 1 on
    it, for 128 x 192 tiles (48 full tiles run as 112 of these), whole rounds plus a half-tile tail (306) and full tiles
    only (135)."""
    from h3_tp2_amd import ops
    a, w, sa, sb = serving_like(M, N, K, seed=3 + M, device=cuda)
    amax = torch.full((M,), 123.0, device=cuda)          # the library zeroes it first
    y = ops.gemm(a, w, sa, sb, torch.bfloat16, row_amax=amax)
    torch.cuda.synchronize()
    assert torch.equal(amax, y.float().abs().amax(dim=1))
    y2, q, s = ops.gemm_quant(a, w, sa, sb)
    torch.cuda.synchronize()
    assert torch.equal(y2.view(torch.int16), y.view(torch.int16))
    assert_quant_equal(q, s, *oracle_quant(y2.cpu()))


@pytest.mark.parametrize("bias", [False, True])
def test_fused_row_amax_fp16_output(cuda, bias):
    """The row maxima of an fp16 output are the fp32 values of its largest rounded entries (not its bits read as
    bf16), with values beyond the bf16-looking range of the fp16 bit patterns (|y| up to ~6e4) and a bias."""
    from h3_tp2_amd import ops
    M, N, K = 700, 1040, 512
    a, w, sa, sb = serving_like(M, N, K, seed=23, device=cuda)
    sa = sa * torch.exp2(torch.randint(-6, 14, (M,), generator=torch.Generator().manual_seed(3))).to(cuda)
    bb = (torch.randn(N, generator=torch.Generator().manual_seed(4)) * 3).to(torch.float16).to(cuda) if bias else None
    amax = torch.full((M,), 5.0, device=cuda)
    y = ops.gemm(a, w, sa, sb, torch.float16, bias=bb, row_amax=amax)
    torch.cuda.synchronize()
    assert torch.equal(amax, y.float().abs().amax(dim=1))
    assert np.array_equal(bits16(ops.gemm(a, w, sa, sb, torch.float16, bias=bb)), bits16(y))


def test_grouped_matches_single(cuda):
    from h3_tp2_amd import ops
    shapes = [(2, 3072, 18432), (512, 4096, 6144), (1600, 1536, 4608), (300, 3072, 1040)]
    probs = []
    for i, (M, K, N) in enumerate(shapes):
        a, w, sa, sb = serving_like(M, N, K, seed=100 + i, device=cuda)
        probs.append((a, w, sa, sb))
    outs = ops.grouped_gemm(probs)
    torch.cuda.synchronize()
    for (a, w, sa, sb), y in zip(probs, outs):
        assert torch.equal(y.view(torch.int16), _gemm(a, w, sa, sb).view(torch.int16))


@pytest.mark.parametrize("shapes", [[(32, 1024, 512), (33, 1024, 512), (1, 256, 4096), (2, 3072, 18432)],
                                    [(2, 3072, 18432), (17, 1536, 4608)]])
def test_grouped_small_groups(cuda, shapes):
    """Groups of at most 32 rows inside the grouped launch (its tiles mostly zero rows) against their single launches,
    which take the small-M form: bit for bit (the same MFMA sequence per element), integer groups against the oracle
    too; a list of small groups only, and the 32 / 33 row boundary."""
    from h3_tp2_amd import ops
    probs = [serving_like(M, N, K, seed=400 + i, device=cuda) for i, (M, K, N) in enumerate(shapes)]
    ints = [int_operands(M, N, K, seed=500 + i, device=cuda) for i, (M, K, N) in enumerate(shapes)]
    outs = ops.grouped_gemm(probs)
    outs_i = ops.grouped_gemm(ints)
    torch.cuda.synchronize()
    for (a, w, sa, sb), y in zip(probs, outs):
        assert torch.equal(y.view(torch.int16), _gemm(a, w, sa, sb).view(torch.int16))
    for (a, w, sa, sb), y in zip(ints, outs_i):
        assert np.array_equal(bits16(y), ref_gemm(a, w, sa, sb))


def test_side_stream_and_scaled_mm_layout(cuda):
    from h3_tp2_amd import ops
    a, w, sa, sb = serving_like(1000, 5376, 7168, seed=5, device=cuda)
    ref = _gemm(a, w, sa, sb)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        y = ops.scaled_mm(a, w.t(), sa.view(-1, 1), sb, torch.bfloat16)     # vLLM's b = w.t()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    assert torch.equal(y.view(torch.int16), ref.view(torch.int16))


def test_rejects_bad_shapes(cuda):
    from h3_tp2_amd import H3Fp8Error, ops
    a = torch.zeros(4, 24, device=cuda, dtype=torch.float8_e4m3fn)
    w = torch.zeros(32, 24, device=cuda, dtype=torch.float8_e4m3fn)
    with pytest.raises(H3Fp8Error):
        ops.gemm(a, w, torch.ones(4, device=cuda), torch.ones(32, device=cuda))     # K % 16 != 0
    raw = torch.zeros(4 * 32 + 1, device=cuda, dtype=torch.uint8)[1:].view(torch.float8_e4m3fn).view(4, 32)
    w2 = torch.zeros(32, 32, device=cuda, dtype=torch.float8_e4m3fn)
    with pytest.raises(H3Fp8Error):
        ops.gemm(raw, w2, torch.ones(4, device=cuda), torch.ones(32, device=cuda))  # misaligned A
    y0 = ops.gemm(a[:0, :16], w[:, :16].contiguous(), torch.ones(0, device=cuda), torch.ones(32, device=cuda))
    assert y0.shape == (0, 32)


@pytest.mark.parametrize("kind,M,N,K", [("serving", 1000, 8192, 5376), ("serving", 333, 3072, 8192),
                                         ("outliers", 2048, 3072, 3072), ("outliers", 1024, 3072, 8192)])
def test_accumulator_error_model(cuda, kind, M, N, K):
    """The raw fp32 accumulator (probe mode, the reference's OUT 0) against the exact sum: within ACC_REL * sum|a w|
    everywhere, and exactly equal on integer operands (exact in any order)."""
    from h3_tp2_amd import ops, synthetic
    if kind == "serving":
        a, w, sa, sb = serving_like(M, N, K, seed=M + N, device=cuda)
    else:
        a, sa = ops.quant_rows(synthetic.activations(M, K, seed=0, n_out=synthetic.n_outliers(K)).to(cuda))
        w, sb = ops.quant_rows(synthetic.weight(N, K, seed=1).to(cuda))
    acc = ops.gemm(a, w, sa, sb, torch.float32).cpu().numpy().astype(np.float64)
    A = O.e4m3_to_f32(bits8(a)).astype(np.float64)
    W = O.e4m3_to_f32(bits8(w)).astype(np.float64)
    err = np.abs(acc - A @ W.T)
    assert (err <= ACC_REL * abs_products(a, w)).all(), float((err / abs_products(a, w)).max())
    ai, wi, sai, sbi = int_operands(300, 528, 768, seed=2, device=cuda)
    acc_i = ops.gemm(ai, wi, sai, sbi, torch.float32).cpu().numpy()
    assert np.array_equal(acc_i, O.matmul_f32(bits8(ai), bits8(wi)))


@pytest.mark.parametrize("M,N,K", [(16740, 9216, 3072), (2048, 3072, 3072), (31248, 3072, 1024)])
def test_half_tile_tail_equals_full_tiles(cuda, M, N, K):
    """A launch whose last round runs as half tiles (256 x 128), or whose whole problem runs as 128 x 192 tiles (2048 x
    3072: 256 of them), gives the same bits as all full tiles (the grouped path never splits): the same MFMA sequence
    per output element.  Also the fused row maxima + quant through the split launch against the oracle's quant of its
    own output."""
    from h3_tp2_amd import ops
    a, w, sa, sb = serving_like(M, N, K, seed=7, device=cuda)
    y = _gemm(a, w, sa, sb)
    (yg,) = ops.grouped_gemm([(a, w, sa, sb)])
    torch.cuda.synchronize()
    assert torch.equal(y.view(torch.int16), yg.view(torch.int16))
    y2, q, s = ops.gemm_quant(a, w, sa, sb)
    torch.cuda.synchronize()
    assert torch.equal(y2.view(torch.int16), y.view(torch.int16))
    assert_quant_equal(q, s, *oracle_quant(y2.cpu()))


@pytest.mark.parametrize("M,N,K", [(4096, 4352, 128), (4100, 4368, 64), (5000, 2560, 64), (2300, 3600, 192),
                                   (1000, 3008, 96), (6000, 2816, 48), (2048, 4096, 64), (300, 400, 176)])
def test_integer_inputs_exact_launch_splits(cuda, M, N, K):
    """Shapes whose tile counts take each launch form on 256 CUs: whole rounds plus a half-tile tail (272, 306 and 264
    tiles), full tiles only (200 and 135 tiles), half tiles only (128 tiles), 128 x 192 tiles (48 full tiles as 128
    of these; 4 as 9, ragged in M, N and K); K below one 128-deep k-step; integer operands, so the output must equal
    the oracle bit for bit, with guard sentinels around it."""
    from h3_tp2_amd import ops
    a, w, sa, sb = int_operands(M, N, K, seed=7 * M + N + K, device=cuda)
    ref = ref_gemm(a, w, sa, sb)
    guard = 4096
    buf = torch.full((M * N + 2 * guard,), float("nan"), device=cuda, dtype=torch.bfloat16)
    buf[:guard] = 7.0
    buf[-guard:] = 7.0
    y = buf[guard:guard + M * N].view(M, N)
    ops.gemm(a, w, sa, sb, torch.bfloat16, out=y)
    torch.cuda.synchronize()
    assert np.array_equal(bits16(y), ref)
    assert bool((buf[:guard] == 7.0).all()) and bool((buf[-guard:] == 7.0).all())
