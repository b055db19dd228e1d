"""Caller-supplied outputs and workspaces are validated before any launch (CPU; no GPU needed).

``ops`` checks the shape, dtype, device and strides of every ``out`` / ``q`` / ``scale`` / ``row_amax`` / ``h_ws`` /
``bias`` a caller hands in: a wrong one must raise ValueError and never reach the C ABI, where it would be an
out-of-bounds device write.  The tests run on CPU tensors with the GPU-only guard switched off and the C call replaced
by a recorder, so a correct call is seen to reach the ABI and a wrong one is seen not to.
"""
import pytest
import torch

from h3_tp2_amd import _lib, ops

E4M3 = torch.float8_e4m3fn
BF16 = torch.bfloat16


@pytest.fixture
def calls(monkeypatch):
    seen = []
    monkeypatch.setattr(ops, "_need_cuda", lambda *ts: None)
    monkeypatch.setattr(ops, "_stream", lambda t: 0)
    monkeypatch.setattr(_lib, "call", lambda name, *args: seen.append(name))
    return seen


def _gemm_operands(M=8, N=32, K=64):
    a = torch.zeros(M, K, dtype=E4M3)
    w = torch.zeros(N, K, dtype=E4M3)
    return a, w, torch.ones(M, 1), torch.ones(N)


def test_quant_rows_buffers(calls):
    x = torch.zeros(8, 64, dtype=BF16)
    ops.quant_rows(x, torch.empty(8, 64, dtype=E4M3), torch.empty(8, 1))
    ops.quant_rows(x, torch.empty(8, 64, dtype=E4M3), torch.empty(8))
    assert calls == ["h3fp8_quant_rows"] * 2
    bad = [
        dict(q=torch.empty(8, 32, dtype=E4M3)),                 # too narrow
        dict(q=torch.empty(4, 64, dtype=E4M3)),                 # too few rows
        dict(q=torch.empty(8, 64, dtype=torch.uint8)),          # wrong dtype
        dict(q=torch.empty(64, 8, dtype=E4M3).t()),             # rows not contiguous
        dict(scale=torch.empty(4, 1)),                          # too few scales
        dict(scale=torch.empty(8, 1, dtype=torch.float16)),     # wrong dtype
        dict(scale=torch.empty(8, 2)[:, :1]),                   # not contiguous
        dict(scale=torch.empty(8, 64)),                         # wrong shape
    ]
    for kw in bad:
        with pytest.raises(ValueError):
            ops.quant_rows(x, **kw)
    assert calls == ["h3fp8_quant_rows"] * 2


def test_quant_rows_amax_buffers(calls):
    x = torch.zeros(8, 64, dtype=BF16)
    ops.quant_rows_amax(x, torch.zeros(8))
    assert calls == ["h3fp8_quant_rows_amax"]
    for amax in (torch.zeros(7), torch.zeros(8, dtype=torch.float64), torch.zeros(16)[::2], torch.zeros(8, 1)):
        with pytest.raises(ValueError):
            ops.quant_rows_amax(x, amax)
    with pytest.raises(ValueError):
        ops.quant_rows_amax(x, torch.zeros(8), q=torch.empty(8, 63, dtype=E4M3))
    with pytest.raises(ValueError):
        ops.quant_rows_amax(x.float(), torch.zeros(8))
    assert calls == ["h3fp8_quant_rows_amax"]


def test_gemm_out_row_amax_bias(calls):
    a, w, sa, sb = _gemm_operands()
    ops.gemm(a, w, sa, sb, BF16, out=torch.empty(8, 32, dtype=BF16), row_amax=torch.zeros(8))
    ops.gemm(a, w, sa, sb, torch.float16, bias=torch.zeros(32, dtype=torch.float16))
    assert calls == ["h3fp8_gemm"] * 2
    bad = [
        dict(out=torch.empty(8, 16, dtype=BF16)),
        dict(out=torch.empty(9, 32, dtype=BF16)),
        dict(out=torch.empty(8, 32, dtype=torch.float16)),       # dtype differs from out_dtype
        dict(out=torch.empty(32, 8, dtype=BF16).t()),
        dict(row_amax=torch.zeros(4)),
        dict(row_amax=torch.zeros(8, dtype=BF16)),
        dict(bias=torch.zeros(16, dtype=BF16)),
        dict(bias=torch.zeros(32)),                              # fp32 bias for a bf16 output
        dict(bias=torch.zeros(64, dtype=BF16)[::2]),
    ]
    for kw in bad:
        with pytest.raises(ValueError):
            ops.gemm(a, w, sa, sb, BF16, **kw)
    assert calls == ["h3fp8_gemm"] * 2


def test_gemm_quant_bias(calls):
    a, w, sa, sb = _gemm_operands()
    ops.gemm_quant(a, w, sa, sb, bias=torch.zeros(32, dtype=BF16))
    with pytest.raises(ValueError):
        ops.gemm_quant(a, w, sa, sb, bias=torch.zeros(31, dtype=BF16))
    with pytest.raises(ValueError):
        ops.gemm_quant(a, w, sa, sb, bias=torch.zeros(32, dtype=torch.float16))
    assert calls == ["h3fp8_gemm_quant"]


def test_gemm_swiglu_bias_and_workspaces(calls):
    a, w, sa, sb = _gemm_operands(M=8, N=64, K=64)          # F = 32
    ops.gemm_swiglu(a, w, sa, sb, bias=torch.zeros(64, dtype=BF16), row_amax=torch.zeros(8))
    ops.gemm_swiglu_quant(a, w, sa, sb, bias=torch.zeros(64, dtype=BF16), h_ws=torch.empty(8, 32, dtype=BF16))
    assert calls == ["h3fp8_gemm_swiglu", "h3fp8_gemm_swiglu_quant"]
    for fn in (ops.gemm_swiglu, ops.gemm_swiglu_quant):
        for bias in (torch.zeros(32, dtype=BF16),            # [F]: the kernel reads 2F entries
                     torch.zeros(64),                         # fp32
                     torch.zeros(64, dtype=torch.float16),
                     torch.zeros(128, dtype=BF16)[::2]):
            with pytest.raises(ValueError):
                fn(a, w, sa, sb, bias=bias)
    with pytest.raises(ValueError):
        ops.gemm_swiglu(a, w, sa, sb, row_amax=torch.zeros(7))
    for hws in (torch.empty(8, 64, dtype=BF16)[:, :32],       # rows of F with a wider stride: the C side assumes F
                torch.empty(8, 31, dtype=BF16), torch.empty(8, 32)):
        with pytest.raises(ValueError):
            ops.gemm_swiglu_quant(a, w, sa, sb, h_ws=hws)
    with pytest.raises(ValueError):
        ops.gemm_swiglu(a, w[:63], sa, sb[:63])               # odd gate/up row count
    assert calls == ["h3fp8_gemm_swiglu", "h3fp8_gemm_swiglu_quant"]


def test_scale_pass_and_consumer_outputs(calls):
    x32 = torch.zeros(8, 32)
    ops.scale_bias_cast(x32, torch.ones(8), torch.ones(32), None, BF16, out=torch.empty(8, 32, dtype=BF16))
    assert calls == ["h3fp8_scale_bias_cast"]
    with pytest.raises(ValueError):
        ops.scale_bias_cast(x32, torch.ones(8), torch.ones(32), None, BF16, out=torch.empty(8, 16, dtype=BF16))
    with pytest.raises(ValueError):
        ops.scale_bias_cast(x32, torch.ones(8), torch.ones(32), torch.zeros(32, dtype=torch.float16), BF16)
    with pytest.raises(ValueError):
        ops.scale_bias_cast(x32, torch.ones(8), torch.ones(32), None, torch.float32)
    x = torch.zeros(8, 32, dtype=BF16)
    gate = torch.zeros(2, 32, dtype=BF16)
    idx = torch.zeros(8, dtype=torch.int64)
    ops.scale_indexed_gate(x32, torch.ones(8), torch.ones(32), None, x, gate, idx, out=torch.empty(8, 32, dtype=BF16))
    with pytest.raises(ValueError):
        ops.scale_indexed_gate(x32, torch.ones(8), torch.ones(32), None, x, gate, idx,
                               out=torch.empty(8, 32, dtype=torch.float16))
    assert calls == ["h3fp8_scale_bias_cast", "h3fp8_scale_indexed_gate"]


def test_swiglu_passes_input_dtype_width_and_bias(calls):
    """scale_swiglu / scale_swiglu_quant read an fp32 [M, 2F] product and a bf16 [2F] bias; silu_mul_quant reads bf16
    [M, 2F].  A wrong input dtype (a bf16 product would be read as fp32: twice its allocation), an odd width or a width
    whose F is not a multiple of 4, and a bias of the wrong dtype or length raise before any launch."""
    x32 = torch.zeros(8, 64)
    sa, sb = torch.ones(8), torch.ones(64)
    ops.scale_swiglu(x32, sa, sb, torch.zeros(64, dtype=BF16))
    ops.scale_swiglu_quant(x32, sa, sb, torch.zeros(64, dtype=BF16))
    ops.silu_mul_quant(torch.zeros(8, 64, dtype=BF16))
    assert calls == ["h3fp8_scale_swiglu", "h3fp8_scale_swiglu_quant", "h3fp8_silu_mul_quant"]
    for fn in (ops.scale_swiglu, ops.scale_swiglu_quant):
        for x in (torch.zeros(8, 64, dtype=BF16),             # a bf16 "product"
                  torch.zeros(8, 64, dtype=torch.float64),
                  torch.zeros(8, 63),                          # odd width
                  torch.zeros(8, 68),                          # F = 34, not a multiple of 4
                  torch.zeros(64, 8).t(),                      # rows not contiguous
                  torch.zeros(8, 2, 32)):                      # not 2-D
            with pytest.raises(ValueError):
                fn(x, sa, torch.ones(x.shape[-1]) if x.dim() == 2 else sb)
        for bias in (torch.zeros(32, dtype=BF16),             # [F]: the kernels read 2F entries
                     torch.zeros(64),                          # fp32
                     torch.zeros(64, dtype=torch.float16),
                     torch.zeros(128, dtype=BF16)[::2]):
            with pytest.raises(ValueError):
                fn(x32, sa, sb, bias)
    for x in (torch.zeros(8, 64), torch.zeros(8, 64, dtype=torch.float16), torch.zeros(8, 63, dtype=BF16),
              torch.zeros(8, 68, dtype=BF16), torch.zeros(8, 68, dtype=BF16)[:, :64], torch.zeros(64, dtype=BF16)):
        with pytest.raises(ValueError):
            ops.silu_mul_quant(x)
    with pytest.raises(ValueError):
        ops.scale_bias_cast(torch.zeros(8, 32, dtype=BF16), torch.ones(8), torch.ones(32), None, BF16)
    assert calls == ["h3fp8_scale_swiglu", "h3fp8_scale_swiglu_quant", "h3fp8_silu_mul_quant"]


def test_mfma_loop_output(calls):
    """The measurement loop writes one float per thread of 256-thread workgroups: its output must be a contiguous
    fp32 tensor of a positive multiple of 256 elements; the FLOP count follows the workgroups and rounds."""
    assert ops.mfma_loop(torch.empty(512), 3) == 2.0 * 32 * 32 * 64 * 16 * 4 * 2 * 3
    assert calls == ["h3fp8_mfma_loop"]
    for out in (torch.empty(300), torch.empty(0), torch.empty(512, dtype=torch.float16), torch.empty(1024)[::2]):
        with pytest.raises(ValueError):
            ops.mfma_loop(out, 3)
    assert calls == ["h3fp8_mfma_loop"]
