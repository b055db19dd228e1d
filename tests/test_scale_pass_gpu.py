"""The two-pass scale pass (``h3fp8_scale_bias_cast``: y = round(sa[m] * (sb[n] * x32[m, n])), bias by one fma) against
the oracle's epilogue, bit for bit: both of its kernels (row segments for a contiguous 16-byte aligned sb, the
elementwise form for strided or unaligned sb), column slices of a wider product (the v columns of the qkv output),
widths that leave a partial segment, bf16 and fp16 outputs with and without a bias, and values pushed to inf."""
import numpy as np
import pytest
import torch

from _util import bits16
from h3_tp2_amd import ops
from oracle import oracle as O

pytestmark = pytest.mark.gpu


def _operands(M, N, seed, out_dtype, bias):
    g = torch.Generator().manual_seed(seed)
    x32 = torch.randn(M, N, generator=g) * 3000
    sa = torch.exp(torch.empty(M).uniform_(-9.0, -2.0, generator=g))
    sb = torch.exp(torch.empty(N).uniform_(-9.5, -7.5, generator=g))
    b = (torch.randn(N, generator=g) * 0.1).to(out_dtype) if bias else None
    return x32, sa, sb, b


def _check(y, x32, sa, sb, b, out_dtype):
    want = O.epilogue(x32.numpy(), sa.numpy(), sb.numpy(), None if b is None else bits16(b),
                      out_fp16=out_dtype == torch.float16)
    got = bits16(y)
    nan = (want & 0x7FFF) > (0x7C00 if out_dtype == torch.float16 else 0x7F80)
    assert np.array_equal((got & 0x7FFF) > (0x7C00 if out_dtype == torch.float16 else 0x7F80), nan)
    bad = (got != want) & ~nan
    assert not bad.any(), f"{int(bad.sum())} values differ, first at {np.argwhere(bad)[:5].tolist()}"


@pytest.mark.parametrize("M,N", [(1, 8), (37, 1000), (300, 3072), (129, 4104), (5, 9216)])
@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("bias", [False, True])
def test_scale_bias_cast_contiguous(cuda, M, N, out_dtype, bias):
    x32, sa, sb, b = _operands(M, N, M * 31 + N, out_dtype, bias)
    y = ops.scale_bias_cast(x32.to(cuda), sa.to(cuda), sb.to(cuda), None if b is None else b.to(cuda), out_dtype)
    _check(y.cpu(), x32, sa, sb, b, out_dtype)


@pytest.mark.parametrize("offset", [0, 8, 6144])
def test_scale_bias_cast_column_slice(cuda, offset):
    """The v columns of a [T, 9216] product into the matching columns of a bf16 placeholder (strided rows in and out;
    offset 8 leaves sb 16-byte aligned only through the slice start, offset 6144 is the qkv layout)."""
    M, W, N = 257, 9216, 3072
    x32, sa, sb, b = _operands(M, W, offset + 1, torch.bfloat16, True)
    xd, sad, sbd, bd = x32.to(cuda), sa.to(cuda), sb.to(cuda), b.to(cuda)
    ph = torch.full((M, W), -1, dtype=torch.int16, device=cuda).view(torch.bfloat16)
    ops.scale_bias_cast(xd[:, offset:offset + N], sad, sbd[offset:offset + N], bd[offset:offset + N], torch.bfloat16,
                        out=ph[:, offset:offset + N])
    host = ph.cpu()
    _check(host[:, offset:offset + N], x32[:, offset:offset + N].contiguous(), sa, sb[offset:offset + N],
           b[offset:offset + N], torch.bfloat16)
    untouched = np.concatenate([bits16(host[:, :offset]).ravel(), bits16(host[:, offset + N:]).ravel()])
    assert (untouched == 0xFFFF).all(), "the pass wrote outside its columns"


def test_scale_bias_cast_strided_and_unaligned_sb(cuda):
    """sb with an element stride (the elementwise kernel) and sb starting 4 bytes past a 16-byte boundary."""
    M, N = 65, 2056
    x32, sa, sb, b = _operands(M, N, 7, torch.bfloat16, True)
    xd, sad = x32.to(cuda), sa.to(cuda)
    sb2 = torch.stack((sb, sb), dim=1).to(cuda)                      # [N, 2]: column 0 has element stride 2
    y = ops.scale_bias_cast(xd, sad, sb2[:, 0], b.to(cuda), torch.bfloat16)
    _check(y.cpu(), x32, sa, sb, b, torch.bfloat16)
    sbp = torch.cat((torch.zeros(1), sb)).to(cuda)[1:]               # 4 bytes past the allocation's start
    y = ops.scale_bias_cast(xd, sad, sbp, b.to(cuda), torch.bfloat16)
    _check(y.cpu(), x32, sa, sb, b, torch.bfloat16)


def test_scale_bias_cast_overflow_and_nan(cuda):
    M, N = 9, 1024
    x32, sa, sb, b = _operands(M, N, 3, torch.bfloat16, False)
    x32[0, :5] = torch.tensor([3e38, -3e38, float("inf"), float("nan"), 0.0])
    sa[1] = 1e30
    sb[7] = float("inf")
    y = ops.scale_bias_cast(x32.to(cuda), sa.to(cuda), sb.to(cuda), None, torch.bfloat16)
    _check(y.cpu(), x32, sa, sb, b, torch.bfloat16)
