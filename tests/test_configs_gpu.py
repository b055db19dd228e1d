"""The benchmark configurations exactly as configured, on the GPU, against the oracle.

* c4 (the 15 s 1344x768 block chain, M = 91 728 tokens): the QKV GEMM (N = 9216) and the gate/up GEMM + SwiGLU +
  requant (F = 8192) at the full token count with integer operands, so every output must equal the oracle bit for bit
  (the accumulator is exact in any order), with guard sentinels around the outputs and the fused row maxima checked.
* The seeded c4 chain (quant -> QKV; attention stand-in -> quant -> out-proj + fused quant -> gate/up + SwiGLU + requant
  -> down + fused quant): every stage's bf16 output equals the oracle's epilogue of that stage's own accumulator (read
  back through the raw-accumulator mode), and every fp8 input equals the oracle's quant of the previous stage's output.
* c5 (the grouped launch with its four groups as configured, the M = 16 740 QKV group included): bit-exact against the
  oracle on integer operands and equal to one GEMM per group on serving-like operands.
* Launches whose activation, scale or output byte ranges exceed 32-bit buffer offsets, so the library runs them as
  several row chunks: integer operands, bit-exact, with the bytes between the output rows as sentinels (pattern of the
  reference's tests/test_fp8_cutlass_gpu.py:58-74).
"""
import numpy as np
import pytest
import torch

from _util import assert_quant_equal, bits8, bits16, f32, int_operands, oracle_quant, ref_gemm, serving_like
from oracle import oracle as O

pytestmark = pytest.mark.gpu

E4M3 = torch.float8_e4m3fn
C4_M = 91728


def _guarded(M, N, dtype, device, fill=7.0, guard=4096):
    buf = torch.full((M * N + 2 * guard,), fill, device=device, dtype=dtype)
    return buf, buf[guard:guard + M * N].view(M, N), guard


def _guards_intact(buf, guard, fill=7.0):
    return bool((buf[:guard] == fill).all()) and bool((buf[-guard:] == fill).all())


def _int_operands_gpu(M, N, K, seed, device):
    """int_operands' distributions with the [M, K] activation and its scales drawn on the GPU (the CPU generator takes
    long at the full c4 size)."""
    a, w, sa, sb = int_operands(1, N, K, seed=seed, device=device)
    g = torch.Generator(device=device).manual_seed(seed)
    a = torch.randint(-4, 5, (M, K), generator=g, device=device).float().to(E4M3)
    sa = torch.exp(torch.empty(M, device=device).uniform_(-9.0, -2.0, generator=g))
    return a, w, sa, sb


def test_c4_qkv_full_size_integer_exact(cuda):
    from h3_tp2_amd import ops
    M, N, K = C4_M, 9216, 3072
    a, w, sa, sb = _int_operands_gpu(M, N, K, seed=41, device=cuda)
    buf, y, guard = _guarded(M, N, torch.bfloat16, cuda)
    amax = torch.full((M,), -1.0, device=cuda)
    ops.gemm(a, w, sa, sb, torch.bfloat16, out=y, row_amax=amax)
    torch.cuda.synchronize()
    assert _guards_intact(buf, guard)
    assert torch.equal(amax, y.float().abs().amax(dim=1))
    ref = ref_gemm(a, w, sa, sb)
    got = bits16(y)
    bad = got != ref
    assert not bad.any(), f"{int(bad.sum())} outputs differ, first at {np.argwhere(bad)[:4].tolist()}"


def test_c4_gate_up_swiglu_requant_full_size_integer_exact(cuda):
    from h3_tp2_amd import _lib, ops
    M, F, K = C4_M, 8192, 3072
    a, w, sa, sb = _int_operands_gpu(M, 2 * F, K, seed=43, device=cuda)
    sb = sb * 40.0                                   # |g|, |u| up to a few units: the SiLU sees both tails
    buf, h, guard = _guarded(M, F, torch.bfloat16, cuda)
    amax = torch.full((M,), -1.0, device=cuda)
    q = torch.empty((M, F), device=cuda, dtype=E4M3)
    s = torch.empty((M,), device=cuda)
    st = torch.cuda.current_stream().cuda_stream
    _lib.call("h3fp8_gemm_swiglu_quant", a.data_ptr(), K, w.data_ptr(), K, sa.data_ptr(), 1, sb.data_ptr(), 1, None,
              M, F, K, h.data_ptr(), amax.data_ptr(), q.data_ptr(), F, s.data_ptr(), st)
    torch.cuda.synchronize()
    assert _guards_intact(buf, guard)
    assert torch.equal(amax, h.float().abs().amax(dim=1))
    acc = O.matmul_f32(bits8(a), bits8(w))
    h_ref = O.scale_swiglu(acc, f32(sa), f32(sb))
    assert np.array_equal(bits16(h), h_ref)
    q_ref, s_ref = O.scale_swiglu_quant(acc, f32(sa), f32(sb))
    del acc
    assert_quant_equal(q, s, q_ref, s_ref)
    # the same kernel through the launcher that allocates its own workspace gives the same bytes
    q2, s2 = ops.gemm_swiglu_quant(a, w, sa, sb)
    torch.cuda.synchronize()
    assert torch.equal(q2.view(torch.uint8), q.view(torch.uint8)) and torch.equal(s2.view(-1), s)


def _rows_sample(M, seed, n=2048):
    """Rows to check against the CPU oracle: the first and last tiles, rows around every 256-row tile edge of the
    first tiles, and a seeded random spread."""
    r = np.random.default_rng(seed)
    edges = np.concatenate([np.arange(0, 600), np.arange(M - 600, M)])
    return np.unique(np.concatenate([edges, r.choice(M, n, replace=False)]))


def _check_stage(y, acc32, sa, sb, rows):
    """bf16 y equals the oracle epilogue of the stage's own fp32 accumulator, on the sampled rows."""
    ref = O.epilogue(f32(acc32[rows]), f32(sa.reshape(-1)[rows]), f32(sb))
    assert np.array_equal(bits16(y[rows]), ref)


def test_c4_chain_stage_by_stage(cuda):
    """The seeded c4 chain as bench.py runs it.  Whole-size properties on the GPU (fused row maxima equal the maxima of
    the stage outputs; the fused quant equals kernel 1 on the stage output); the oracle (the epilogue of the stage's
    accumulator, then the quant) on a row sample of every stage."""
    from h3_tp2_amd import ops, synthetic
    c = synthetic.CONFIGS["c4_chain_1344x768_15s"]
    M, K, F = c["M"], c["K"], 8192
    rows = torch.from_numpy(_rows_sample(M, seed=4)).to(cuda)

    def wq(n, k, seed):
        w, s = ops.quant_rows(synthetic.weight(n, k, seed).to(cuda))
        return w, s.view(-1)

    wqkv, sqkv = wq(3 * K, K, 1)
    wo, so = wq(K, K, 4)
    wgu, sgu = wq(2 * F, K, 2)
    wd, sd = wq(K, F, 3)
    x = synthetic.activations(M, K, seed=0, n_out=c["n_out"]).to(cuda)
    xo = synthetic.activations(M, K, seed=5, n_out=c["n_out"]).to(cuda)

    def quant_matches(x_bf16, q, s):
        xr = x_bf16[rows]
        qr, sr = oracle_quant(xr.cpu())
        assert_quant_equal(q.view(torch.uint8)[rows], s.reshape(-1)[rows], qr, sr)

    q0, s0 = ops.quant_rows(x)
    quant_matches(x, q0, s0)
    yqkv = ops.gemm(q0, wqkv, s0, sqkv)
    _check_stage(yqkv, ops.gemm(q0, wqkv, s0, sqkv, torch.float32), s0, sqkv, rows)
    del yqkv

    qo, so_ = ops.quant_rows(xo)
    y_out, qg, sg = ops.gemm_quant(qo, wo, so_, so)
    _check_stage(y_out, ops.gemm(qo, wo, so_, so, torch.float32), so_, so, rows)
    quant_matches(y_out, qg, sg)
    q_k1, s_k1 = ops.quant_rows(y_out)                # the fused quant equals kernel 1 on the whole output
    assert torch.equal(qg.view(torch.uint8), q_k1.view(torch.uint8)) and torch.equal(sg, s_k1)
    del y_out, q_k1

    hws = torch.empty((M, F), device=cuda, dtype=torch.bfloat16)
    qh, sh = ops.gemm_swiglu_quant(qg, wgu, sg, sgu, h_ws=hws)
    acc_gu = ops.gemm(qg, wgu, sg, sgu, torch.float32)
    acc_rows = f32(acc_gu[rows])
    del acc_gu
    assert np.array_equal(bits16(hws[rows]), O.scale_swiglu(acc_rows, f32(sg.reshape(-1)[rows]), f32(sgu)))
    q_ref, s_ref = O.scale_swiglu_quant(acc_rows, f32(sg.reshape(-1)[rows]), f32(sgu))
    assert_quant_equal(qh.view(torch.uint8)[rows], sh.reshape(-1)[rows], q_ref, s_ref)
    q_k1, s_k1 = ops.quant_rows(hws)
    assert torch.equal(qh.view(torch.uint8), q_k1.view(torch.uint8)) and torch.equal(sh, s_k1)
    del hws, q_k1

    y_d, qn, sn = ops.gemm_quant(qh, wd, sh, sd)
    _check_stage(y_d, ops.gemm(qh, wd, sh, sd, torch.float32), sh, sd, rows)
    quant_matches(y_d, qn, sn)
    torch.cuda.synchronize()


C5 = [(2, 3072, 18432), (512, 4096, 6144), (1600, 1536, 4608), (16740, 3072, 9216)]


def test_c5_grouped_as_configured_integer_exact(cuda):
    from h3_tp2_amd import ops
    probs = [int_operands(M, N, K, seed=200 + i, device=cuda) for i, (M, K, N) in enumerate(C5)]
    outs = ops.grouped_gemm(probs)
    torch.cuda.synchronize()
    for (a, w, sa, sb), y in zip(probs, outs):
        assert np.array_equal(bits16(y), ref_gemm(a, w, sa, sb))


def test_c5_grouped_as_configured_equals_single(cuda):
    from h3_tp2_amd import ops
    probs = [serving_like(M, N, K, seed=300 + i, device=cuda) for i, (M, K, N) in enumerate(C5)]
    outs = ops.grouped_gemm(probs)
    singles = [ops.gemm(a, w, sa, sb) for a, w, sa, sb in probs]
    torch.cuda.synchronize()
    for y, y1 in zip(outs, singles):
        assert torch.equal(y.view(torch.int16), y1.view(torch.int16))


# ---- launches split into row chunks (32-bit buffer offsets) ----------------------------------------------------------
# M = 33 000 rows, K = 128, N = 256, with the activation rows 65 536 bytes apart, the per-token scales 20 000 floats
# apart and the output rows 40 000 elements apart: each range exceeds what one launch can address, and the library
# cuts the launch at 26 624 rows (bf16 output; 13 312 for the fp32 accumulator).  Everything between the rows that the
# kernel may read or write is poisoned: NaN fp8 codes and NaN scales that no output may pick up, sentinels that no
# store may touch.

SPLIT_M, SPLIT_K, SPLIT_N, LDA, SA_STRIDE, LDY = 33000, 128, 256, 65536, 20000, 40000


def _strided_operands(cuda, seed):
    a_c, w, sa_c, sb = int_operands(SPLIT_M, SPLIT_N, SPLIT_K, seed=seed, device=cuda)
    abuf = torch.full((SPLIT_M, LDA), 0x7F, device=cuda, dtype=torch.uint8)      # 0x7f: e4m3fn NaN
    abuf[:, :SPLIT_K] = a_c.view(torch.uint8)
    a = abuf.view(E4M3)[:, :SPLIT_K]
    sbuf = torch.full((SPLIT_M * SA_STRIDE,), float("nan"), device=cuda)
    sbuf[::SA_STRIDE] = sa_c
    sa = sbuf[::SA_STRIDE]
    return a, a_c, w, sa, sa_c, sb


@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float32])
def test_split_launch_offsets_exact(cuda, out_dtype):
    from h3_tp2_amd import ops
    a, a_c, w, sa, sa_c, sb = _strided_operands(cuda, seed=17)
    assert a.stride(0) == LDA and sa.stride(0) == SA_STRIDE
    ybuf = torch.full((SPLIT_M, LDY), 7.0, device=cuda, dtype=out_dtype)
    y = ybuf[:, :SPLIT_N]
    amax = torch.full((SPLIT_M,), -1.0, device=cuda) if out_dtype == torch.bfloat16 else None
    ops.gemm(a, w, sa, sb, out_dtype, out=y, row_amax=amax)
    torch.cuda.synchronize()
    assert bool((ybuf[:, SPLIT_N:] == 7.0).all()), "a store landed between the output rows"
    acc = O.matmul_f32(bits8(a_c), bits8(w))
    if out_dtype == torch.float32:
        assert np.array_equal(f32(y), acc)
    else:
        assert np.array_equal(bits16(y), O.epilogue(acc, f32(sa_c), f32(sb)))
        assert torch.equal(amax, y.float().abs().amax(dim=1))


def test_split_launch_swiglu_exact(cuda):
    """Kernel 3 with the h rows 40 000 elements apart (the launch is cut at 26 624 rows)."""
    from h3_tp2_amd import _lib
    F = SPLIT_N // 2
    a, a_c, w, sa, sa_c, sb = _strided_operands(cuda, seed=19)
    sb = sb * 40.0
    hbuf = torch.full((SPLIT_M, LDY), 7.0, device=cuda, dtype=torch.bfloat16)
    amax = torch.full((SPLIT_M,), -1.0, device=cuda)
    _lib.call("h3fp8_gemm_swiglu", a.data_ptr(), LDA, w.data_ptr(), SPLIT_K, sa.data_ptr(), SA_STRIDE, sb.data_ptr(), 1,
              None, hbuf.data_ptr(), LDY, amax.data_ptr(), SPLIT_M, F, SPLIT_K, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    h = hbuf[:, :F]
    assert bool((hbuf[:, F:] == 7.0).all()), "a store landed between the h rows"
    acc = O.matmul_f32(bits8(a_c), bits8(w))
    assert np.array_equal(bits16(h), O.scale_swiglu(acc, f32(sa_c), f32(sb)))
    assert torch.equal(amax, h.float().abs().amax(dim=1))
