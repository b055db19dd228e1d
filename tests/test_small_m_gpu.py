"""The small-M form of kernel 2 (M <= 32 token rows: one wave per 16 weight rows, the weight streamed through a private
LDS ring).

* Bit-identity with the tiled kernel: the same MFMA sequence per output element (weight row at A-row n % 32, token at
  B-column m % 32, 64-deep k chunks ascending, zero chunks past K), so the M-row product equals rows 0..M-1 of the
  tiled kernel's product of a 64-row operand whose first M rows are the same.  Checked on random serving-like and
  outlier operands (where the MFMA's inexact accumulation would expose any change of order), for bf16 / fp16 outputs,
  bias, the row maxima of the fused quant, scalar scales and the raw fp32 accumulator.
* Integer operands: exact against the oracle, with guard sentinels around the output (no write outside [M, N]).
* The adaLN modulation shape of the grouped workload (M = 2, K = 3072, N = 6 x 3072) and K tails (K mod 128 != 0).
"""
import numpy as np
import pytest
import torch

from _util import bits16, f32, int_operands, ref_gemm, serving_like
from h3_tp2_amd import synthetic

pytestmark = pytest.mark.gpu

E4M3 = torch.float8_e4m3fn


def _outlier_operands(M, N, K, seed, device):
    """N(0,1) activations with x40 outlier channels and N(0,0.02) weights, quantised by kernel 1 on the GPU."""
    from h3_tp2_amd import ops
    x = synthetic.activations(M, K, seed=seed, n_out=3).to(device)
    w = synthetic.weight(N, K, seed=seed + 1).to(device)
    a, sa = ops.quant_rows(x)
    wq, sw = ops.quant_rows(w)
    return a, wq, sa.view(-1), sw.view(-1)


def _tiled_rows(a, w, sa, sb, M, **kw):
    """Rows 0..M-1 of the tiled kernel's product: the operand padded to 64 rows (M > 32 takes the tiled form)."""
    from h3_tp2_amd import ops
    pad = 64 - M
    g = torch.Generator().manual_seed(M)
    a64 = torch.cat([a, torch.randint(-8, 9, (pad, a.shape[1]), generator=g).float().to(E4M3).to(a.device)])
    sa64 = torch.cat([sa.reshape(-1), torch.full((pad,), 1e-3, device=sa.device)]) if sa.numel() > 1 else sa
    amax = kw.pop("row_amax", None)
    amax64 = torch.zeros(64, device=a.device) if amax is not None else None
    y = ops.gemm(a64, w, sa64, sb, row_amax=amax64, **kw)
    torch.cuda.synchronize()
    return y[:M], (amax64[:M] if amax is not None else None)


@pytest.mark.parametrize("M,N,K", [(1, 256, 3072), (2, 18432, 3072), (5, 528, 1040), (17, 4608, 1536),
                                   (31, 6144, 4096), (32, 3072, 8192), (3, 16, 16), (32, 48, 80)])
def test_small_m_equals_tiled_kernel_random(cuda, M, N, K):
    from h3_tp2_amd import ops
    for a, w, sa, sb in (serving_like(M, N, K, seed=M + N, device=cuda), _outlier_operands(M, N, K, 7 * M, cuda)):
        y = ops.gemm(a, w, sa, sb)
        torch.cuda.synchronize()
        ref, _ = _tiled_rows(a, w, sa, sb, M)
        assert np.array_equal(bits16(y), bits16(ref))


# (7, 1040, 2048): 65 waves, plain weight loads; (2, 16400, 1024): 1025 waves, at least 4 per CU, so the weight loads
# take the non-temporal hint
@pytest.mark.parametrize("M,N,K", [(7, 1040, 2048), (2, 16400, 1024)])
@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("bias", [False, True])
@pytest.mark.parametrize("amax", [False, True])
def test_small_m_epilogue_forms_equal_tiled(cuda, out_dtype, bias, amax, M, N, K):
    from h3_tp2_amd import ops
    a, w, sa, sb = _outlier_operands(M, N, K, 3, cuda)
    bb = (torch.randn(N, generator=torch.Generator().manual_seed(2)) * 0.3).to(out_dtype).to(cuda) if bias else None
    am = torch.full((M,), -1.0, device=cuda) if amax else None
    y = ops.gemm(a, w, sa, sb, out_dtype, bb, row_amax=am)
    torch.cuda.synchronize()
    ref, ref_am = _tiled_rows(a, w, sa, sb, M, out_dtype=out_dtype, bias=bb, row_amax=am)
    assert y.dtype == out_dtype and np.array_equal(bits16(y), bits16(ref))
    if amax:
        assert np.array_equal(f32(am).view(np.uint32), f32(ref_am).view(np.uint32))
        # the row maxima are max |y| of the rounded outputs
        assert np.array_equal(f32(am), np.abs(f32(y).astype(np.float32)).max(axis=1))


def test_small_m_scalar_scales_and_raw_accumulator(cuda):
    from h3_tp2_amd import ops
    M, N, K = 9, 768, 3072
    a, w, sa, sb = _outlier_operands(M, N, K, 11, cuda)
    s1 = sa[:1].reshape(())
    y = ops.gemm(a, w, s1, sb[:1].reshape(1, 1))
    torch.cuda.synchronize()
    ref, _ = _tiled_rows(a, w, s1, sb[:1].reshape(1, 1), M)
    assert np.array_equal(bits16(y), bits16(ref))
    acc = ops.gemm(a, w, sa, sb, torch.float32)
    torch.cuda.synchronize()
    acc_ref, _ = _tiled_rows(a, w, sa, sb, M, out_dtype=torch.float32)
    assert np.array_equal(f32(acc).view(np.uint32), f32(acc_ref).view(np.uint32))


@pytest.mark.parametrize("M,N,K", [(1, 16, 16), (2, 18432, 3072), (32, 272, 1040), (13, 1024, 336), (32, 64, 8192)])
def test_small_m_integer_exact_with_guards(cuda, M, N, K):
    from h3_tp2_amd import ops
    a, w, sa, sb = int_operands(M, N, K, seed=M * 3 + K, device=cuda)
    ref = ref_gemm(a, w, sa, sb)
    guard = 2048
    buf = torch.full((M * N + 2 * guard,), float("nan"), device=cuda, dtype=torch.bfloat16)
    buf[:guard] = 7.0
    buf[-guard:] = 7.0
    y = buf[guard:guard + M * N].view(M, N)
    ops.gemm(a, w, sa, sb, torch.bfloat16, out=y)
    torch.cuda.synchronize()
    assert np.array_equal(bits16(y), ref)
    assert bool((buf[:guard] == 7.0).all()) and bool((buf[-guard:] == 7.0).all())


def test_small_m_strided_output_rows(cuda):
    """An output with a row stride larger than N: the columns between N and the stride stay untouched."""
    from h3_tp2_amd import ops
    M, N, K, ld = 4, 96, 256, 136
    a, w, sa, sb = int_operands(M, N, K, seed=5, device=cuda)
    full = torch.full((M, ld), 3.0, device=cuda, dtype=torch.bfloat16)
    ops.gemm(a, w, sa, sb, torch.bfloat16, out=full[:, :N])
    torch.cuda.synchronize()
    assert np.array_equal(bits16(full[:, :N]), ref_gemm(a, w, sa, sb))
    assert bool((full[:, N:] == 3.0).all())
