"""The per-token quant of the out projection's input read straight from the Ulysses receive buffer [P, M, hl, d]
(``h3fp8_quant_segments``) against the oracle's quant of the unpacked rows, bit for bit.

Follows the reference's tests/test_fp8_quant_fuse_gpu.py:84-90 (receive buffers with per-row log-normal magnitudes,
M = 1 / 200 / 4100) and tests/test_ulysses_outq_gpu.py (P = 1 / 2 / 4 segments, the contiguous-row layout, zero and
non-finite rows).
"""
import numpy as np
import pytest
import torch

from _util import assert_quant_equal, bits16
from oracle import oracle as O

pytestmark = pytest.mark.gpu
BF16 = torch.bfloat16


def _recv(P, M, hl, d, seed):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(P, M, hl, d, generator=g) * torch.exp(torch.randn(1, M, 1, 1, generator=g))).to(BF16)


@pytest.mark.parametrize("P,hl,d", [(2, 28, 128), (1, 24, 128), (4, 6, 128), (2, 12, 128)])
@pytest.mark.parametrize("M", [1, 200, 4100])
def test_quant_from_recv(cuda, P, hl, d, M):
    from h3_tp2_amd import fp8_quant_fuse as fq, ops
    recv = _recv(P, M, hl, d, seed=M + P)
    if M > 3:
        recv[:, 1] = 0.0                                   # a zero row: the minimum scale
        recv[1 % P, 2, 0, 5] = float("nan")                # NaN in one segment of row 2
        recv[0, 3, 1, 0] = float("inf")
    rows = recv.transpose(0, 1).reshape(M, P * hl * d)     # the unpacked out-projection input
    q_ref, s_ref = O.quant_rows(bits16(rows))
    rd = recv.to(cuda)
    q, s = ops.quant_from_recv(rd)
    torch.cuda.synchronize()
    assert q.shape == (M, P * hl * d) and s.shape == (M, 1)
    assert_quant_equal(q, s, q_ref, s_ref)
    q2, s2 = fq.unpack_quant(rd)
    torch.cuda.synchronize()
    assert_quant_equal(q2, s2, q_ref, s_ref)
    un = fq.unpack_stock(rd, P * hl)
    torch.cuda.synchronize()
    assert np.array_equal(bits16(un[0].reshape(M, -1)), bits16(rows))


def test_quant_rows_contiguous_and_strided_layouts(cuda):
    """The same entry point on ordinary rows (stride_m = P * seg) and on rows with a stride past their width."""
    from h3_tp2_amd import ops
    M, P, seg, pad = 300, 2, 1536, 64
    g = torch.Generator().manual_seed(3)
    x = (torch.randn(M, P * seg + pad, generator=g) * 3).to(BF16)
    q_ref, s_ref = O.quant_rows(bits16(x[:, :P * seg].contiguous()))
    xd = x.to(cuda)
    q, s = ops.quant_segments(xd, M, P, seg, seg, P * seg + pad)
    torch.cuda.synchronize()
    assert_quant_equal(q, s, q_ref, s_ref)


def test_argument_errors(cuda):
    from h3_tp2_amd import _lib, ops
    x = torch.zeros(4, 100, dtype=BF16, device=cuda)
    with pytest.raises(_lib.H3Fp8Error, match="multiples of 8"):
        ops.quant_segments(x, 4, 1, 100, 0, 100)
    with pytest.raises(ValueError, match="past the source"):
        ops.quant_segments(x, 4, 2, 96, 400, 96)
    q, s = ops.quant_segments(x, 0, 2, 96, 0, 96)
    assert q.shape == (0, 192)
