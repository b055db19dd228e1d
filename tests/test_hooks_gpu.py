"""GPU tests of the hook surface: the install checks pass, the dispatcher's two levels agree bit for bit, the QuantFP8
drop-in and the SwiGLU stash path give the oracle's bytes through the real kernels."""
import numpy as np
import pytest
import torch

from _util import assert_quant_equal, bits16, bits8, int_operands, oracle_quant, serving_like
from h3_tp2_amd import fp8_gemm, fp8_quant_fuse, fp8_swiglu
from oracle import oracle as O

pytestmark = pytest.mark.gpu
BF16 = torch.bfloat16


def test_dispatcher_install_check(cuda):
    assert fp8_gemm.selfcheck(cuda) == []


def test_swiglu_install_check(cuda):
    assert fp8_swiglu.probe_gemm_swiglu(cuda)


@pytest.mark.parametrize("M,N,K", [(1, 256, 3072), (4100, 5376, 7168), (333, 1040, 1024)])
def test_fused_equals_two_pass_bitwise(cuda, M, N, K):
    """Kernel 2 with the epilogue in registers equals its raw fp32 product + the scale pass bit for bit (same
    accumulator: same tile order and K order in both modes)."""
    a, w, sa, sb = serving_like(M, N, K, seed=M + N, device=cuda)
    b = w.t()
    y1 = fp8_gemm.scaled_mm_fused(a, b, sa.view(M, 1), sb, BF16)
    y2 = fp8_gemm.scaled_mm_tensor32(a, b, sa.view(M, 1), sb, BF16)
    assert np.array_equal(bits16(y1), bits16(y2))
    bias = (torch.randn(N, generator=torch.Generator().manual_seed(1)) * 0.1).to(torch.float16).to(cuda)
    y1 = fp8_gemm.scaled_mm_fused(a, b, sa, sb, torch.float16, bias)
    y2 = fp8_gemm.scaled_mm_tensor32(a, b, sa, sb, torch.float16, bias)
    assert np.array_equal(bits16(y1), bits16(y2))


def test_dispatcher_end_to_end(cuda, monkeypatch):
    class Ops:
        def __init__(self):
            self.stock_calls = 0

        def cutlass_scaled_mm(self, *args):
            self.stock_calls += 1
            return None

    fake = Ops()
    fake.cutlass_scaled_mm = fake.cutlass_scaled_mm
    monkeypatch.setattr(fp8_gemm, "_state", dict(fp8_gemm._state))
    assert fp8_gemm.install(fake, level="hip", check=True)
    a, w, sa, sb = int_operands(200, 400, 512, seed=3, device=cuda)
    y = fake.cutlass_scaled_mm(a, w.t(), sa.view(-1, 1), sb, BF16)
    acc = a.float() @ w.float().t()
    ref = ((sb.view(1, -1) * acc) * sa.view(-1, 1)).to(BF16)
    assert torch.equal(y.view(torch.int16), ref.view(torch.int16)) and fake.stock_calls == 0


def test_quantfp8_dropin_kernel1(cuda, monkeypatch):
    class QuantFP8:
        static = False
        use_per_token_if_dynamic = True
        is_group_quant = False
        num_token_padding = None

        def forward(self, x, scale=None, scale_ub=None):
            raise AssertionError("stock quant called for an eligible input")

    monkeypatch.setattr(fp8_quant_fuse, "_state", dict(fp8_quant_fuse._state))
    fp8_quant_fuse.install((), quant_cls=QuantFP8)
    g = torch.Generator().manual_seed(5)
    x = (torch.randn(1000, 3072, generator=g) * 3).to(BF16)
    x[:, 7] *= 40
    q, s = QuantFP8().forward(x.to(cuda))
    q_ref, s_ref = oracle_quant(x)
    assert_quant_equal(q, s, q_ref, s_ref)
    assert q.shape == (1000, 3072) and s.shape == (1000, 1)


def test_silu_mul_quant_site_matches_oracle(cuda):
    g = torch.Generator().manual_seed(6)
    x = (torch.randn(300, 2 * 1024, generator=g) * 2).to(BF16)
    q, s = fp8_quant_fuse.silu_mul_quant(x.to(cuda))
    q_ref, s_ref = O.quant_rows(O.swiglu_bf16(bits16(x)))
    assert_quant_equal(q, s, q_ref, s_ref)
    assert bits8(q).shape == (300, 1024)
