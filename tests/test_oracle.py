"""Pins of the CPU oracle (CPU only): every oracle function is checked against something it was not derived from --
torch's and numpy's own casts and arithmetic, the golden fixtures of tests/golden/ (written by make_golden.py from
torch's CPU routines in the reference mirrors' order), the known answers of the reference's tests, brute force on the
e4m3 grid, exact rational / integer arithmetic, and invariants that a dropped term or a swapped operand breaks."""
import os

import numpy as np
import pytest
import torch

from oracle import oracle as O

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
E4M3 = torch.float8_e4m3fn


def golden(name):
    return np.load(os.path.join(GOLDEN, name))


def f32_from_bits(u):
    return np.asarray(u, dtype=np.uint32).view(np.float32)


def sweep_patterns(n_random=1 << 21, seed=0):
    """fp32 bit patterns: random, every special class, and the rounding boundaries of bf16/fp16/e4m3."""
    rng = np.random.default_rng(seed)
    r = rng.integers(0, 1 << 32, n_random, dtype=np.uint64).astype(np.uint32)
    hi = rng.integers(0, 1 << 16, 4096, dtype=np.uint64).astype(np.uint32) << 16
    lows = np.array([0x0000, 0x0001, 0x7FFF, 0x8000, 0x8001, 0xFFFF], np.uint32)
    bnd = (hi[:, None] | lows[None, :]).reshape(-1)
    spec = np.array([0, 0x80000000, 0x7F800000, 0xFF800000, 0x7FC00000, 0xFFC00000, 0x7F800001, 0x00000001,
                     0x007FFFFF, 0x00800000, 0x7F7FFFFF, 0xFF7FFFFF], np.uint32)
    return np.concatenate([r, bnd, spec])


# ---- casts ----------------------------------------------------------------------------------------------------------

def test_min_scale_constant():
    assert np.float32(O.MIN_SCALE).view(np.uint32) == 0x36924925
    assert O.lib().oracle_min_scale() == pytest.approx(4.359654212748865e-06, rel=1e-7)


def test_bf16_rne_matches_torch_cast():
    u = sweep_patterns()
    x = f32_from_bits(u)
    ours = O.bf16_rne(x)
    ref = torch.from_numpy(x.copy()).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    nan = np.isnan(x)
    assert np.array_equal(ours[~nan], ref[~nan])
    assert np.all((ours[nan] & 0x7F80) == 0x7F80) and np.all(ours[nan] & 0x007F)


def test_fp16_rne_matches_numpy_cast():
    u = sweep_patterns(seed=1)
    x = f32_from_bits(u)
    ours = O.fp16_rne(x)
    with np.errstate(over="ignore"):
        ref = x.astype(np.float16).view(np.uint16)
    nan = np.isnan(x)
    assert np.array_equal(ours[~nan], ref[~nan])
    assert np.all(np.isnan(ours[nan].view(np.float16)))


def test_e4m3_decode_every_code():
    codes = np.arange(256, dtype=np.uint8)
    ours = O.e4m3_to_f32(codes)
    ref = torch.from_numpy(codes).view(E4M3).float().numpy()
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(ours), nan) and nan.sum() == 2
    assert np.array_equal(ours[~nan].view(np.uint32), ref[~nan].view(np.uint32))


def test_e4m3_encode_matches_torch_cast_dense():
    # every 37th fp32 pattern below 512 in magnitude (both signs) plus the general sweep
    base = np.arange(0, 0x44000000, 37, dtype=np.uint32)
    u = np.concatenate([base, base | 0x80000000, sweep_patterns(seed=2)])
    x = f32_from_bits(u)
    ours = O.e4m3fn_from_f32(x)
    ref = torch.from_numpy(x.copy()).to(E4M3).view(torch.uint8).numpy()
    nan = (ref & 0x7F) == 0x7F
    assert np.array_equal((ours & 0x7F) == 0x7F, nan)
    assert np.array_equal(ours[~nan], ref[~nan])


def test_e4m3_encode_brute_force_nearest_even():
    """Nearest grid value by exhaustive search over the 253 finite codes, ties to the even code."""
    rng = np.random.default_rng(3)
    x = np.concatenate([rng.uniform(-448, 448, 20000), rng.uniform(-0.02, 0.02, 20000),
                        rng.uniform(-1e-3, 1e-3, 5000)]).astype(np.float32)
    grid_codes = np.array([c for c in range(256) if (c & 0x7F) != 0x7F], np.uint8)
    grid = O.e4m3_to_f32(grid_codes).astype(np.float64)
    d = np.abs(x.astype(np.float64)[:, None] - grid[None, :])
    best = d.min(1, keepdims=True)
    cand = d == best
    # among tied candidates: the even mantissa code (lowest bit 0); +0 preferred for sign of zero by the value's sign
    pick = np.empty(len(x), np.uint8)
    for i in range(len(x)):
        cs = grid_codes[cand[i]]
        if len(cs) > 1:
            cs = cs[(cs & 1) == 0] if np.any((cs & 1) == 0) else cs
            if len(cs) > 1:                                  # +0 / -0: sign of x
                cs = cs[(cs & 0x80) == (0x80 if np.signbit(x[i]) else 0)]
        pick[i] = cs[0]
    ours = O.e4m3fn_from_f32(x)
    assert np.array_equal(ours, pick)


def test_e4m3_grid_idempotent():
    codes = np.array([c for c in range(256) if (c & 0x7F) != 0x7F], np.uint8)
    assert np.array_equal(O.e4m3fn_from_f32(O.e4m3_to_f32(codes)), codes)


# ---- per-token quant ------------------------------------------------------------------------------------------------

def test_quant_matches_golden():
    gd = golden("quant.npz")
    q, s = O.quant_rows(gd["x"])
    assert np.array_equal(s.view(np.uint32), gd["scale"].view(np.uint32))
    assert np.array_equal(q, gd["q"])
    assert s[3] == O.MIN_SCALE and not q[3].any()               # the all-zero row


def test_quant_every_bf16_row_maximum():
    """Every positive finite bf16 as a row maximum: scale = max(amax / 448, MIN_SCALE) with IEEE division (numpy),
    and the whole row against the golden sweep (torch's ops)."""
    gd = golden("amax_sweep.npz")
    q, s = O.quant_rows(gd["x"])
    amax = (gd["x"][:, 0].astype(np.uint32) << 16).view(np.float32)
    want = np.maximum(amax / np.float32(448.0), O.MIN_SCALE)
    assert np.array_equal(s.view(np.uint32), want.view(np.uint32))
    assert np.array_equal(s.view(np.uint32), gd["scale"].view(np.uint32))
    assert np.array_equal(q, gd["q"])
    big = amax / np.float32(448.0) >= O.MIN_SCALE
    assert np.all(q[big, 0] == 0x7E) and np.all(q[big, 1] == 0xFE)   # the maximum lands on +-448


def test_quant_uses_reciprocal_multiply():
    """x * (1/scale), not x / scale: find rows where the two differ and check the oracle takes the reciprocal form."""
    rng = np.random.default_rng(5)
    x = (rng.standard_normal((4000, 64)) * np.exp(rng.standard_normal((4000, 1)) * 2)).astype(np.float32)
    xb = O.bf16_rne(x)
    q, s = O.quant_rows(xb)
    xf = O.bf16_to_f32(xb)
    inv = np.float32(1.0) / s[:, None]
    by_recip = O.e4m3fn_from_f32(np.clip(xf * inv, -448, 448))
    by_div = O.e4m3fn_from_f32(np.clip(xf / s[:, None], -448, 448))
    assert (by_recip != by_div).any()                         # the sample distinguishes the two forms
    assert np.array_equal(q, by_recip)


def test_quant_invariants():
    rng = np.random.default_rng(6)
    x = (rng.standard_normal((500, 256)) * np.exp(rng.standard_normal((500, 1)) * 3)).astype(np.float32)
    xb = O.bf16_rne(x)
    q, s = O.quant_rows(xb)
    qn, sn = O.quant_rows(xb ^ 0x8000)                       # negation flips the sign bit only
    assert np.array_equal(sn, s)
    nz = (q & 0x7F) != 0
    assert np.array_equal(qn[nz], q[nz] ^ 0x80)
    dec = O.e4m3_to_f32(q)
    assert np.all(np.abs(dec) <= 448)
    xf = O.bf16_to_f32(xb)
    err = np.abs(dec * s[:, None] - xf)
    assert np.all(err <= np.abs(xf) * 2.0 ** -4 + s[:, None] * 2.0 ** -10)   # half an e4m3 ulp (+ subnormal step)


def test_quant_nonfinite_rows():
    row_inf = np.zeros((1, 16), np.float32)
    row_inf[0, :3] = [np.inf, 1.0, -1.0]
    row_nan = np.ones((1, 16), np.float32)
    row_nan[0, 5] = np.nan
    q, s = O.quant_rows(O.bf16_rne(np.concatenate([row_inf, row_nan])))
    assert np.isinf(s[0]) and (q[0, 0] & 0x7F) == 0x7F          # inf * (1/inf) = NaN
    assert q[0, 1] == 0x00 and q[0, 2] == 0x80                   # finite * 0 = +-0
    assert np.isnan(s[1]) and np.all((q[1] & 0x7F) == 0x7F)


def test_quant_matches_torch_formula_random():
    """The reference's quant_torch (fp8_quant_fuse.py:302-307) in torch ops on seeded bf16 rows."""
    g = torch.Generator().manual_seed(7)
    h = (torch.randn(300, 1000, generator=g) * torch.exp(torch.randn(300, 1, generator=g) * 3)).to(torch.bfloat16)
    h[::37] = 0
    amax = h.abs().max(dim=-1)[0].unsqueeze(-1).float()
    scale = (amax / 448.0).clamp(min=O.MIN_SCALE.item())
    ref = (h.float() * scale.reciprocal()).clamp(-448.0, 448.0).to(E4M3).view(torch.uint8).numpy()
    q, s = O.quant_rows(h.view(torch.int16).numpy().view(np.uint16))
    assert np.array_equal(q, ref) and np.array_equal(s, scale.numpy().reshape(-1))


# ---- epilogue -------------------------------------------------------------------------------------------------------

def test_epilogue_matches_golden():
    gd = golden("epilogue.npz")
    assert np.array_equal(O.epilogue(gd["acc"], gd["sa"], gd["sb"]), gd["y_bf16"])
    assert np.array_equal(O.epilogue(gd["acc"], gd["sa"], gd["sb"], out_fp16=True), gd["y_fp16"])
    assert np.array_equal(O.epilogue(gd["acc"], gd["sa"], gd["sb"], gd["bias"]), gd["y_bias_bf16"])


def test_epilogue_order_known_answer():
    """tests/test_fp8_gemm.py:67-75 of the reference: (sb * x) * sa, which differs from (x * sa) * sb here."""
    x = np.array([[1.0000001192092896]], np.float32)
    sa, sb = np.array([3.0], np.float32), np.array([0.1], np.float32)
    right = (sb[0] * x[0, 0]) * sa[0]
    assert O.epilogue(x, sa, sb, out_fp16=True)[0, 0] == np.float16(right).view(np.uint16)
    assert O.bf16_rne(np.full((1, 1), right, np.float32))[0, 0] == O.epilogue(x, sa, sb)[0, 0]
    # cases where the order survives the final rounding: the oracle must give (sb * acc) * sa on every one
    rng = np.random.default_rng(11)
    n = 1 << 21
    acc = rng.standard_normal(n).astype(np.float32) * 100
    s_a = np.exp(rng.uniform(-9, -2, n)).astype(np.float32)
    s_b = np.exp(rng.uniform(-9, -7, n)).astype(np.float32)
    right = (s_b * acc) * s_a
    naive = (acc * s_a) * s_b
    for fp16 in (True, False):
        cast = O.fp16_rne if fp16 else O.bf16_rne
        idx = np.nonzero(cast(right) != cast(naive))[0]
        assert len(idx) >= 5
        for i in idx[:200]:
            y = O.epilogue(acc[i:i + 1].reshape(1, 1), s_a[i:i + 1], s_b[i:i + 1], out_fp16=fp16)
            assert y[0, 0] == cast(right[i:i + 1])[0]


# ---- SiLU / SwiGLU --------------------------------------------------------------------------------------------------

def test_silu_table_against_float64_and_torch_exp():
    tab = O.silu_table()
    g = O.bf16_to_f32(np.arange(65536, dtype=np.uint32).astype(np.uint16))
    with np.errstate(over="ignore", invalid="ignore"):
        e = np.exp(-g.astype(np.float64)).astype(np.float32)          # correctly rounded fp32 exp
        s = g / (np.float32(1.0) + e)
    ref = O.bf16_rne(s.astype(np.float32))
    nan = np.isnan(g)
    assert np.array_equal(tab[~nan], ref[~nan])
    assert np.all((tab[nan] & 0x7F80) == 0x7F80)
    # the reference's CPU mirror uses torch's fp32 exp, which is not correctly rounded in general; on the 65536 bf16
    # gate values it gives the same silu after the bf16 rounding everywhere (NaN outputs compared as NaN)
    torch_tab = golden("swiglu.npz")["silu_torch_exp"]
    t_nan = ((torch_tab & 0x7F80) == 0x7F80) & ((torch_tab & 0x7F) != 0)
    o_nan = ((tab & 0x7F80) == 0x7F80) & ((tab & 0x7F) != 0)
    assert np.array_equal(t_nan, o_nan) and o_nan.sum() == 254 + 1      # 254 NaN gates and silu(-inf) = -inf / inf
    assert np.array_equal(tab[~o_nan], torch_tab[~o_nan])


def test_swiglu_matches_golden_directed():
    gd = golden("swiglu.npz")
    h = O.scale_swiglu(gd["x32"], gd["sa"], gd["sb"])
    want = gd["h"]
    nan = (want & 0x7F80) == 0x7F80
    nan &= (want & 0x7F) != 0
    assert np.array_equal((h & 0x7F80) == 0x7F80, (want & 0x7F80) == 0x7F80)
    assert np.array_equal(h[~nan], want[~nan])


def test_swiglu_negative_zero_up():
    # gate 1 (silu > 0) with up = -0 -> +0; gate -1 (silu < 0) with up = +-0 -> -0
    gu = O.bf16_rne(np.array([[1.0, -1.0, -0.0, -0.0], [1.0, -1.0, 0.0, 0.0]], np.float32))
    h = O.swiglu_bf16(gu)
    assert h.tolist() == [[0x0000, 0x8000], [0x0000, 0x8000]]


def test_scale_swiglu_quant_is_composition():
    rng = np.random.default_rng(8)
    acc = (rng.standard_normal((40, 512)) * 50).astype(np.float32)
    sa = np.exp(rng.uniform(-3, 0, 40)).astype(np.float32)
    sb = np.exp(rng.uniform(-3, 0, 512)).astype(np.float32)
    q, s = O.scale_swiglu_quant(acc, sa, sb)
    q2, s2 = O.quant_rows(O.scale_swiglu(acc, sa, sb))
    assert np.array_equal(q, q2) and np.array_equal(s, s2)
    h = O.scale_swiglu(acc, sa, sb)
    gu = O.epilogue(acc, sa, sb)
    assert np.array_equal(h, O.swiglu_bf16(gu))


# ---- product --------------------------------------------------------------------------------------------------------

def test_dequant_matmul_exact_on_integers():
    rng = np.random.default_rng(9)
    a = rng.integers(-4, 5, (37, 256)).astype(np.float32)
    w = rng.integers(-2, 3, (29, 256)).astype(np.float32)
    ac, wc = O.e4m3fn_from_f32(a), O.e4m3fn_from_f32(w)
    exact = (a.astype(np.int64) @ w.astype(np.int64).T).astype(np.float32)
    assert np.array_equal(O.dequant_matmul(ac, wc), exact)
    assert np.array_equal(O.matmul_f32(ac, wc), exact)


def test_dequant_matmul_k_ascending_fp32():
    rng = np.random.default_rng(10)
    ac = rng.integers(0, 256, (8, 96)).astype(np.uint8)
    wc = rng.integers(0, 256, (5, 96)).astype(np.uint8)
    ac[(ac & 0x7F) == 0x7F] = 0
    wc[(wc & 0x7F) == 0x7F] = 0
    a, w = O.e4m3_to_f32(ac), O.e4m3_to_f32(wc)
    ref = np.zeros((8, 5), np.float32)
    for k in range(96):                                   # fp32, one rounding per multiply and per add, k ascending
        ref = (ref + (a[:, k:k + 1] * w[None, :, k]).astype(np.float32)).astype(np.float32)
    assert np.array_equal(O.dequant_matmul(ac, wc), ref)



# ---- the producers with the quant fused in (RMSNorm + AdaLN modulation -> per-token quant) ---------------------------

from _util import bits16, mod_inputs, standin_gate_rms, standin_rms  # noqa: E402

BF16 = torch.bfloat16


def _bf(vals):
    return bits16(torch.as_tensor(vals, dtype=torch.float32).to(BF16))


def test_row_sumsq_is_the_exact_sum():
    """Rows whose squares span few binades: the fp64 sum is exact in any order, so the oracle's total equals math.fsum
    of the exact squares; rows whose squares span ~50 binades: the fp64 sum rounds, its fp32 rounding is still the
    correctly rounded sum."""
    import math
    rng = np.random.default_rng(3)
    for H in (8, 64, 520, 5376, 8192):
        for spread in (1.0, 4.0):
            x = (rng.standard_normal(H) * np.exp(rng.standard_normal(H) * spread)).astype(np.float32)
            xb = O.bf16_rne(x)
            xf = O.bf16_to_f32(xb).astype(np.float64)
            exact = math.fsum(v * v for v in xf)
            s = O.row_sumsq(xb)
            if spread == 1.0:
                assert s == exact
            assert np.float32(s) == np.float32(exact)


def test_rms_constant_rows_closed_form():
    """x_k = c, weight 1, shift 0, scale 0, eps 0: var = c^2, r = 1 / |c|, h = sign(c) exactly (c * fl(1/|c|) rounds
    to +-1 in bf16 for every bf16 c); weight 2 doubles it.  A wrong divisor (H), a dropped rsqrt or a swapped operand
    gives another value."""
    for H in (8, 64, 1000, 5376):
        cs = np.array([1.0, -1.0, 2.0 ** -60, 3.0, -7.5, 1e10, 0.3, -1e-20], np.float32)
        x = np.repeat(_bf(cs)[:, None], H, axis=1)
        M = x.shape[0]
        zeros = np.zeros((1, H), np.uint16)
        for w, want in ((1.0, 1.0), (2.0, 2.0)):
            h, q, s = O.rms_quant(x, _bf(np.full(H, w)), zeros, zeros, np.zeros(M, np.int64), 0.0)
            ref = _bf(np.sign(cs)[:, None] * want * np.ones((1, H)))
            assert np.array_equal(h, ref), (H, w)


def test_rms_zero_rows_give_shift():
    """x = 0: var = 0, r = 1/sqrt(eps), every product is +-0, so h = bf16(+-0 + shift) = shift for nonzero shift."""
    H = 256
    x = np.zeros((3, H), np.uint16)
    rng = np.random.default_rng(4)
    sh = _bf(rng.standard_normal((2, H)) + 0.01)
    sc = _bf(rng.standard_normal((2, H)))
    h, q, s = O.rms_quant(x, _bf(np.ones(H)), sh, sc, np.array([1, 0, 1]), 1e-6)
    assert np.array_equal(h, sh[[1, 0, 1]])


def test_rms_power_of_two_scale_invariance():
    """eps = 0: scaling a row by 2^k scales var by 4^k, sqrt by 2^k and r by 2^-k exactly, so h, q and the scale do
    not change."""
    x, w, sh, sc, _, idx = mod_inputs(16, 1024, seed=5)
    base = O.rms_quant(bits16(x), bits16(w), bits16(sh), bits16(sc), idx.numpy(), 0.0)
    for k in (-20, -3, 5, 30):
        xs = (x.float() * 2.0 ** k).to(BF16)
        out = O.rms_quant(bits16(xs), bits16(w), bits16(sh), bits16(sc), idx.numpy(), 0.0)
        for a, b in zip(base, out):
            assert np.array_equal(a, b), k


def test_rms_modulation_order_known_answer():
    """A row that normalises to exactly 3 (constant 4.0, weight 3, eps 0): h = bf16(3 * (1 + scale) + shift) with each
    fp32 operation rounded -- numpy's fp32 arithmetic; swapping shift and scale changes it."""
    H = 512
    rng = np.random.default_rng(6)
    sh = _bf(rng.standard_normal((1, H)) * 3)
    sc = _bf(rng.standard_normal((1, H)) * 3)
    x = np.repeat(_bf([4.0])[:, None], H, axis=1)
    h, _, _ = O.rms_quant(x, _bf(np.full(H, 3.0)), sh, sc, np.zeros(1, np.int64), 0.0)
    g = np.float32(1.0) + O.bf16_to_f32(sc[0]).astype(np.float32)
    o = np.float32(3.0) * g + O.bf16_to_f32(sh[0]).astype(np.float32)
    assert np.array_equal(h[0], O.bf16_rne(o.astype(np.float32)))
    swapped = np.float32(3.0) * (np.float32(1.0) + O.bf16_to_f32(sh[0])) + O.bf16_to_f32(sc[0])
    assert not np.array_equal(h[0], O.bf16_rne(swapped.astype(np.float32)))


def test_rms_index_mapping():
    """Row m uses table row indices[m]: each row equals the same computation with that table row alone at index 0."""
    x, w, sh, sc, _, idx = mod_inputs(12, 256, seed=7, B=5)
    h, q, s = O.rms_quant(bits16(x), bits16(w), bits16(sh), bits16(sc), idx.numpy(), 1e-6)
    for m in range(12):
        i = int(idx[m])
        h1, q1, s1 = O.rms_quant(bits16(x[m:m + 1]), bits16(w), bits16(sh[i:i + 1]), bits16(sc[i:i + 1]),
                                 np.zeros(1, np.int64), 1e-6)
        assert np.array_equal(h[m], h1[0]) and np.array_equal(q[m], q1[0]) and s[m] == s1[0]


def _check_against_standin(x, h, h_ref, w, sc, idx, eps):
    """Rows whose fp32 sum of squares is the same in both: bit-identical modulated rows (every other operation is the
    same fp32 arithmetic).  Rows where torch's fp32 sum differs from the correctly rounded one: r moves by a few fp32
    ulps, so each element within one bf16 ulp plus 2^-20 of |n * (1 + scale)|."""
    xf = x.float()
    torch_ss = (xf * xf).sum(dim=1).numpy()
    ours = np.array([np.float32(O.row_sumsq(r)) for r in bits16(x)])
    same = torch_ss.view(np.uint32) == ours.view(np.uint32)
    assert same.mean() > 0.5
    assert np.array_equal(h[same], bits16(h_ref)[same])
    if (~same).any():
        var = (xf * xf).sum(dim=1, keepdim=True) / x.shape[1]
        big = (xf * torch.rsqrt(var + eps) * w.float() * (1.0 + sc.index_select(0, idx).float())).abs().numpy()
        a, b = O.bf16_to_f32(h).astype(np.float64), O.bf16_to_f32(bits16(h_ref)).astype(np.float64)
        tol = np.maximum(np.abs(a), np.abs(b)) * 2.0 ** -7 + big * 2.0 ** -20
        assert (np.abs(a - b) <= tol)[~same].all()


@pytest.mark.parametrize("H", [1024, 5376])
def test_rms_matches_the_torch_standin(H):
    """torch's CPU evaluation of the stock producer (tests/fake_h3_consumers.py:77-84); q / scale are quant_rows of h."""
    x, w, sh, sc, _, idx = mod_inputs(200, H, seed=H)
    h, q, s = O.rms_quant(bits16(x), bits16(w), bits16(sh), bits16(sc), idx.numpy(), 1e-6)
    _check_against_standin(x, h, standin_rms(x, w, sh, sc, idx, 1e-6), w, sc, idx, 1e-6)
    q2, s2 = O.quant_rows(h)
    assert np.array_equal(q, q2) and np.array_equal(s.view(np.uint32), s2.view(np.uint32))


def test_gate_rms_residual_and_composition():
    """residual_out = bf16(residual + gate[i] * branch) equals torch's CPU stand-in bit for bit; h / q / scale equal
    rms_quant applied to residual_out; the modulated row agrees with the stand-in's as in the plain form."""
    H = 3072
    x, w, sh, sc, gt, idx = mod_inputs(150, H, seed=8)
    br = (torch.randn(150, H, generator=torch.Generator().manual_seed(9)) * 3).to(BF16)
    ro, h, q, s = O.gate_rms_quant(bits16(x), bits16(gt), bits16(br), bits16(w), bits16(sh), bits16(sc), idx.numpy(),
                                   1e-6)
    r_ref, h_ref = standin_gate_rms(x, gt, br, w, sh, sc, idx, 1e-6)
    assert np.array_equal(ro, bits16(r_ref))
    h2, q2, s2 = O.rms_quant(ro, bits16(w), bits16(sh), bits16(sc), idx.numpy(), 1e-6)
    assert np.array_equal(h, h2) and np.array_equal(q, q2) and np.array_equal(s.view(np.uint32), s2.view(np.uint32))
    _check_against_standin(r_ref, h, h_ref, w, sc, idx, 1e-6)


def test_rms_nonfinite_rows():
    """A NaN in a row makes var NaN: every h of the row is NaN.  An infinity makes var infinite and r = 0: that element
    is inf * 0 = NaN, the others +-0 + shift = shift.  Both rows get a NaN scale and NaN codes where h is NaN."""
    x, w, sh, sc, _, idx = mod_inputs(4, 64, seed=10)
    xb = bits16(x).copy()
    xb[1, 3] = 0x7FC0
    xb[2, 5] = 0x7F80
    h, q, s = O.rms_quant(xb, bits16(w), bits16(sh), bits16(sc), idx.numpy(), 1e-6)
    nan = (h & 0x7FFF) > 0x7F80
    assert nan[1].all() and np.isnan(s[1]) and ((q[1] & 0x7F) == 0x7F).all()
    assert nan[2, 5] and nan[2].sum() == 1 and np.isnan(s[2]) and (q[2, 5] & 0x7F) == 0x7F
    shift2 = bits16(sh)[int(idx[2])]
    keep = np.arange(64) != 5
    nz = (shift2 & 0x7FFF) != 0
    assert np.array_equal(h[2][keep & nz], shift2[keep & nz])
    assert np.isfinite(s[[0, 3]]).all()


# ---- the consumer of the qkv output: qk-RMSNorm + RoPE (head_dim 128, rotary 96) --------------------------------------

from _util import rope_table, standin_qk_norm_rope  # noqa: E402


def _heads(T, Hh, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    mag = torch.exp(torch.randn(T, Hh, 1, generator=g))
    return (torch.randn(T, Hh, 128, generator=g) * mag * scale).to(BF16)


def test_qk_norm_rope_rotation_closed_forms():
    """cos = 1, sin = 0 passes the normalised row through; cos = 0, sin = 1 rotates it by a quarter turn:
    out[d] = -n[d + 48] (d < 48), n[d - 48] (48 <= d < 96), n[d] (d >= 96).  A constant head of a power of two with
    eps = 0 and weight 1 normalises to exactly +-1."""
    T, Hh = 5, 3
    x = _heads(T, Hh, seed=1)
    w = (1.0 + 0.1 * torch.randn(128, generator=torch.Generator().manual_seed(2))).to(BF16)
    ident = np.concatenate([np.ones((T, 48)), np.zeros((T, 48))], axis=1).astype(np.float32)
    quarter = np.concatenate([np.zeros((T, 48)), np.ones((T, 48))], axis=1).astype(np.float32)
    n = O.qk_norm_rope(bits16(x), bits16(w), ident, 1e-6)
    r = O.qk_norm_rope(bits16(x), bits16(w), quarter, 1e-6)
    want = n.copy()
    want[..., :48] = n[..., 48:96] ^ 0x8000
    want[..., 48:96] = n[..., :48]
    assert np.array_equal(r, want)
    c = torch.full((T, Hh, 128), -0.25).to(BF16)
    c[1] = 8.0
    out = O.qk_norm_rope(bits16(c), _bf(np.ones(128)), ident, 0.0)
    assert np.array_equal(out[0], np.full((Hh, 128), 0xBF80, np.uint16)) and (out[1] == 0x3F80).all()


def test_qk_norm_rope_scale_invariance():
    """eps = 0: a head scaled by 2^k normalises to the same bf16 values, so the rotated output does not change."""
    T, Hh = 4, 2
    x = _heads(T, Hh, seed=3)
    w = (1.0 + 0.1 * torch.randn(128, generator=torch.Generator().manual_seed(4))).to(BF16)
    tab = rope_table(T, torch.float32).numpy()
    base = O.qk_norm_rope(bits16(x), bits16(w), tab, 0.0)
    for k in (-12, 7):
        assert np.array_equal(O.qk_norm_rope(bits16((x.float() * 2.0 ** k).to(BF16)), bits16(w), tab, 0.0), base)


@pytest.mark.parametrize("rope_dtype", [torch.float32, torch.bfloat16])
def test_qk_norm_rope_matches_the_torch_standin(rope_dtype):
    """torch's CPU evaluation of the stock kernel's stand-in: heads whose fp32 sums of squares agree are bit-identical
    (every other operation is the same fp32 arithmetic); the others within one bf16 ulp plus 2^-20 of the rotated
    terms."""
    T, Hh = 64, 6
    x = _heads(T, Hh, seed=5)
    w = (1.0 + 0.1 * torch.randn(128, generator=torch.Generator().manual_seed(6))).to(BF16)
    tab = rope_table(T, rope_dtype)
    out = O.qk_norm_rope(bits16(x), bits16(w), tab.float().numpy(), 1e-6)
    ref = bits16(standin_qk_norm_rope(x, w, tab, 1e-6))
    xf = x.float()
    torch_ss = (xf * xf).sum(dim=-1).numpy()
    ours = np.array([[np.float32(O.row_sumsq(bits16(x[t, h]))) for h in range(Hh)] for t in range(T)])
    same = torch_ss.view(np.uint32) == ours.view(np.uint32)
    assert same.mean() > 0.5
    assert np.array_equal(out[same], ref[same])
    a, b = O.bf16_to_f32(out).astype(np.float64), O.bf16_to_f32(ref).astype(np.float64)
    big = np.abs(O.bf16_to_f32(out)).max(axis=-1, keepdims=True) * 3
    tol = np.maximum(np.abs(a), np.abs(b)) * 2.0 ** -7 + big * 2.0 ** -7
    assert (np.abs(a - b) <= tol)[~same].all()


def test_qk_head_sum_order_is_pinned():
    """The order-sensitive head: the oracle's normalised output equals the one computed from the kernel's lane order's
    sum and differs from a 32 x 4 order's (so the GPU comparison against the oracle pins the kernel's order)."""
    from _util import CONTIG32_LANES, KERNEL_LANES, ORDER_DIM, ORDER_HEAD, ORDER_W, lane_order_sumsq
    x = np.zeros(128, np.float32)
    for d, v in ORDER_HEAD.items():
        x[d] = v
    s8, s32 = lane_order_sumsq(x, KERNEL_LANES), lane_order_sumsq(x, CONTIG32_LANES)
    assert s8 != s32
    w = np.ones(128, np.float32)
    w[ORDER_DIM] = ORDER_W
    ident = np.concatenate([np.ones((1, 48)), np.zeros((1, 48))], axis=1).astype(np.float32)
    out = O.qk_norm_rope(O.bf16_bits_from_f32(x).reshape(1, 1, 128), O.bf16_bits_from_f32(w), ident, 1e-6)

    def norm(var):
        v = np.float32(np.float32(var) / np.float32(128.0))
        r = np.float32(1.0) / np.sqrt(np.float32(v + np.float32(1e-6)))
        return O.bf16_bits_from_f32(np.array([np.float32(x[ORDER_DIM] * r) * np.float32(ORDER_W)], np.float32))[0]
    assert out[0, 0, ORDER_DIM] == norm(s8)
    assert norm(s8) != norm(s32)


# ---- the torch restatement of the reference's CPU path (the CPU baseline leg of bench.py) ---------------------------
from oracle import torch_path as TP  # noqa: E402


def test_torch_path_quant_equals_the_oracle():
    """quant_torch's torch ops give the C oracle's fp8 bytes and scales: seeded rows with outlier channels, the golden
    fixture's rows, a zero row (MIN_SCALE) and inf / NaN rows."""
    g = torch.Generator().manual_seed(31)
    x = torch.randn(257, 3072, generator=g) * torch.exp(torch.randn(257, 1, generator=g) * 1.5)
    x[:, :3] *= 40.0
    x[5] = 0.0
    x[7, 11] = float("inf")
    x[9, 100] = float("nan")
    gold = np.load(os.path.join(os.path.dirname(__file__), "golden", "quant.npz"))
    for xb in (x.to(torch.bfloat16), torch.from_numpy(gold["x"].view(np.int16)).view(torch.bfloat16)):
        q, s = TP.quant(xb)
        qr, sr = O.quant_rows(xb.view(torch.int16).numpy().view(np.uint16))
        nan_q = (qr & 0x7F) == 0x7F
        qb = q.view(torch.uint8).numpy()
        assert np.array_equal((qb & 0x7F) == 0x7F, nan_q) and np.array_equal(qb[~nan_q], qr[~nan_q])
        sv = s.view(-1).numpy()
        assert np.array_equal(np.isnan(sv), np.isnan(sr))
        ok = ~np.isnan(sr)
        assert np.array_equal(sv[ok].view(np.uint32), sr[ok].view(np.uint32))


def test_torch_path_epilogue_and_swiglu_equal_the_oracle():
    """epilogue_torch / swiglu_epilogue_torch's torch ops on one fp32 accumulator give the C oracle's bits (the SiLU
    through torch's CPU exp, which agrees with the correctly rounded exp on every bf16 gate)."""
    g = torch.Generator().manual_seed(32)
    M, F = 193, 640
    acc = torch.randn(M, 2 * F, generator=g) * 2000
    acc[3, :5] = torch.tensor([0.0, -0.0, 1e-30, -1e-30, 3e4])
    sa = torch.rand(M, generator=g) * 1e-3 + 1e-4
    sb = torch.rand(2 * F, generator=g) * 1e-2 + 1e-3
    y = TP.epilogue(acc, sa, sb)
    assert np.array_equal(y.view(torch.int16).numpy().view(np.uint16), O.epilogue(acc.numpy(), sa.numpy(), sb.numpy()))
    h = TP.swiglu(acc, sa, sb)
    assert np.array_equal(h.view(torch.int16).numpy().view(np.uint16), O.scale_swiglu(acc.numpy(), sa.numpy(),
                                                                                     sb.numpy()))


def test_torch_path_product_exact_on_integers():
    g = torch.Generator().manual_seed(33)
    a = torch.randint(-4, 5, (64, 256), generator=g).float().to(torch.float8_e4m3fn)
    w = torch.randint(-2, 3, (96, 256), generator=g).float().to(torch.float8_e4m3fn)
    acc = TP.product(a, w)
    assert np.array_equal(acc.numpy(), O.dequant_matmul(a.view(torch.uint8).numpy(), w.view(torch.uint8).numpy()))
