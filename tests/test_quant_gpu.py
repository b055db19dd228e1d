"""Kernel 1 (per-token dynamic e4m3fn quant) against the oracle, bit for bit (fp8 bytes and scale bits).

Cases follow the reference's tests: tests/test_fp8_quant_fuse_gpu.py:114-134 (directed rows, every positive finite bf16
as a row maximum), tests/test_fp8_quant_fuse.py:367-377 (zero row -> MIN_SCALE), plus widths of every register
configuration of the kernel, ragged M, strided rows, non-finite rows and the measured activations at full size.
"""
import numpy as np
import pytest
import torch

from _util import assert_quant_equal, bits16, oracle_quant

pytestmark = pytest.mark.gpu

BF16 = torch.bfloat16


def _run(x, dev):
    from h3_tp2_amd import ops
    xd = x.to(dev)
    q, s = ops.quant_rows(xd)
    torch.cuda.synchronize()
    return q, s


def test_hw_e4m3_conversion_matches_torch_rule(cuda):
    """Every fp32 bit pattern in [-448, 448] and every NaN through the hardware cvt vs the software rule."""
    from h3_tp2_amd import ops
    bad, nan_bad = ops.selfcheck_e4m3()
    assert bad == 0 and nan_bad == 0, (bad, nan_bad)


def test_hw_bf16_conversion_matches_rne(cuda):
    """The epilogues' hardware fp32 -> bf16 pair conversion equals the RNE rule on all 2^32 fp32 patterns."""
    from h3_tp2_amd import ops
    assert ops.selfcheck_bf16() == (0, 0)


@pytest.mark.parametrize("M,K", [(1, 16), (3, 512), (200, 3072), (333, 5376), (64, 8192), (17, 14336), (5, 20480),
                                 (1000, 1536), (31, 4096), (7, 1040), (129, 7168), (2, 18432)])
@pytest.mark.parametrize("kind", ["normal", "lognormal"])
def test_quant_matches_oracle(cuda, M, K, kind):
    from h3_tp2_amd import synthetic
    x = synthetic.activations(M, K, seed=M * 31 + K, n_out=synthetic.n_outliers(K), kind=kind)
    q, s = _run(x, cuda)
    assert q.dtype == torch.float8_e4m3fn and q.shape == (M, K) and s.shape == (M, 1) and s.dtype == torch.float32
    assert_quant_equal(q, s, *oracle_quant(x))


def test_quant_directed_rows(cuda):
    """The reference's directed rows (tests/test_fp8_quant_fuse_gpu.py:114-126) at K = 5376."""
    K = 5376
    g = torch.Generator().manual_seed(3)
    rows = [torch.zeros(K), torch.full((K,), -0.0)]
    r = torch.zeros(K); r[17] = 1e-38; rows.append(r)
    rows.append(torch.randn(K, generator=g) * 1e-30)
    r = torch.randn(K, generator=g); r[5] = 3.0e38; rows.append(r)
    rows.append(torch.linspace(-448, 448, K))
    rows.append(torch.randn(K, generator=g) * 1e4)
    x = torch.stack(rows).to(BF16)
    q, s = _run(x, cuda)
    q_ref, s_ref = oracle_quant(x)
    assert_quant_equal(q, s, q_ref, s_ref)
    # zero rows: the minimum scale 1/(448*512) (tests/test_fp8_quant_fuse.py:367-377)
    assert s_ref[0] == np.float32(1.0 / (448.0 * 512.0)) and s_ref[1] == s_ref[0]


def test_quant_exhaustive_row_maximum(cuda):
    """Every positive finite bf16 value as a row maximum, its negation in the row, uniform entries below it
    (tests/test_fp8_quant_fuse_gpu.py:121-134)."""
    bits = torch.arange(1, 0x7F80, dtype=torch.int32)
    amax = bits.to(torch.int16).view(BF16)
    n, K = amax.numel(), 1024
    g = torch.Generator().manual_seed(7)
    h = ((torch.rand(n, K, generator=g) * 2 - 1) * amax.float()[:, None]).to(BF16)
    h[:, 0] = amax
    h[:, 1] = -amax
    q, s = _run(h, cuda)
    assert_quant_equal(q, s, *oracle_quant(h))


@pytest.mark.parametrize("M", [7, 16387])
def test_quant_nonfinite_rows(cuda, M):
    """NaN / inf in a row: in the first and in the second half of the row (K = 3072 splits a row over two waves that
    exchange their maxima; an odd row count leaves the last workgroup half empty), and in a row whose other half holds
    the largest finite value; the same rows again as the last ones."""
    K = 3072
    x = torch.randn(M, K, generator=torch.Generator().manual_seed(1))
    for base in sorted({0, M - 7}):
        x[base + 0, 10] = float("nan")
        x[base + 1, 20] = float("inf")
        x[base + 2, 30] = -float("inf")
        x[base + 4, K - 20] = float("nan")
        x[base + 5, K - 30] = -float("inf")
        x[base + 6, 5] = 3.0e38
        x[base + 6, K - 1] = float("inf")
    x = x.to(BF16)
    q, s = _run(x, cuda)
    assert_quant_equal(q, s, *oracle_quant(x))
    for base in sorted({0, M - 7}):
        assert torch.isnan(s[base]).item() and torch.isinf(s[base + 1]).item()
        assert torch.isnan(s[base + 4]).item() and torch.isinf(s[base + 5]).item() and torch.isinf(s[base + 6]).item()


def test_quant_strided_rows_and_empty(cuda):
    from h3_tp2_amd import ops
    wide = torch.randn(100, 3072 + 64, generator=torch.Generator().manual_seed(2)).to(BF16)
    x = wide[:, :3072]
    q, s = ops.quant_rows(wide.to(cuda)[:, :3072])                          # row stride 3136, K 3072
    torch.cuda.synchronize()
    assert_quant_equal(q, s, *oracle_quant(x.contiguous()))
    q0, s0 = ops.quant_rows(torch.empty((0, 3072), device=cuda, dtype=BF16))
    assert q0.shape == (0, 3072) and s0.shape == (0, 1)


@pytest.mark.parametrize("M,K", [(257, 8192), (3, 3072), (129, 3000), (64, 4096), (33, 6144), (5, 8200),
                                 (7, 16384), (2, 1536), (9, 512)])
def test_quant_rows_amax_tail(cuda, M, K):
    """The tail pass with the row maxima given equals the full quant: one wave per row (K <= 2560) and a row split over
    two waves (3 .. 16 chunks per lane each), odd row counts (half of the last workgroup idle) and ragged widths."""
    from h3_tp2_amd import ops
    x = torch.randn(M, K, generator=torch.Generator().manual_seed(4 + K)).to(BF16)
    x[0, K - 1] = 300.0                                 # the maximum in the row's last chunk (the second wave's part)
    amax = x.float().abs().amax(dim=1)
    guard = 4096
    buf = torch.full((M * K + 2 * guard,), 0x5a, dtype=torch.uint8, device=cuda)
    q = buf[guard:guard + M * K].view(M, K)
    s = torch.full((M + 1,), -1.0, device=cuda)
    rc = ops.quant_rows_amax(x.to(cuda), amax.to(cuda), q=q.view(torch.float8_e4m3fn), scale=s[:M].view(M, 1))
    torch.cuda.synchronize()
    assert_quant_equal(rc[0], rc[1], *oracle_quant(x))
    assert bool((buf[:guard] == 0x5a).all()) and bool((buf[-guard:] == 0x5a).all())
    assert float(s[M]) == -1.0


def test_quant_rejects_bad_arguments(cuda):
    from h3_tp2_amd import H3Fp8Error, ops
    with pytest.raises(H3Fp8Error):
        ops.quant_rows(torch.empty((4, 12), device=cuda, dtype=BF16))          # K not a multiple of 8
    with pytest.raises(ValueError):
        ops.quant_rows(torch.empty((4, 16), device=cuda, dtype=torch.float16))


@pytest.mark.parametrize("name", ["c1_single_linear", "c2_qkv_960x576_5s", "c3_ffn_1344x768_5s"])
def test_quant_measured_activations_full_size(cuda, name):
    from h3_tp2_amd import synthetic
    c = synthetic.CONFIGS[name]
    x = synthetic.activations(c["M"], c["K"], seed=0, n_out=c["n_out"])
    q, s = _run(x, cuda)
    assert_quant_equal(q, s, *oracle_quant(x))
