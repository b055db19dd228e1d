"""The per-token quant fused into its producers (RMSNorm + AdaLN modulation; gated residual + RMSNorm + AdaLN
modulation) against the oracle, bit for bit: fp8 bytes, scale bits, the modulated bf16 row (placeholder mode) and
residual_out.

Follows the reference's tests/test_fp8_quant_fuse_gpu.py:40-80 (serving-like magnitudes, [B, 6H] modulation tables
read through chunk views, M = 1 / 200 / 1000 / 4100, both placeholder modes) plus ragged widths, int32 / strided
indices and directed rows (zero, NaN, inf, subnormal, overflowing squares, an index out of range).
"""
import numpy as np
import pytest
import torch

from _util import assert_quant_equal, bits16, mod_inputs
from oracle import oracle as O

pytestmark = pytest.mark.gpu
BF16 = torch.bfloat16
EPS = 1e-6


def _nan_aware_equal(out_bits: np.ndarray, ref_bits: np.ndarray, what: str):
    nan_ref = (ref_bits & 0x7FFF) > 0x7F80
    assert np.array_equal((out_bits & 0x7FFF) > 0x7F80, nan_ref), f"{what}: NaN positions differ"
    bad = (out_bits != ref_bits) & ~nan_ref
    assert not bad.any(), f"{what}: {int(bad.sum())} bf16 values differ, first at {np.argwhere(bad)[:5].tolist()}"


def _tables(dev, *views):
    """The modulation-table views on the device with their row stride kept: the [B, 6H] tensor they slice is moved
    once and sliced again there (``.to`` of a view would make it contiguous)."""
    base = views[0]._base
    assert base is not None and all(v._base is base for v in views)
    bd = base.to(dev)
    H = views[0].shape[1]
    out = []
    for v in views:
        off = v.storage_offset() - base.storage_offset()
        out.append(bd[:, off:off + H])
        assert out[-1].stride(0) == 6 * H
    return out


def _directed(x: torch.Tensor) -> torch.Tensor:
    """Rows 0-5 of x replaced by: zeros, a NaN, an inf, subnormals, squares that overflow fp32, one huge outlier."""
    x = x.clone()
    M, H = x.shape
    if M < 6:
        return x
    x[0] = 0.0
    x[1, H // 3] = float("nan")
    x[2, H - 1] = float("inf")
    x[3] = torch.full((H,), 1e-39).to(BF16) * torch.sign(x[3].float() + 0.5).to(BF16)
    x[4, :4] = 2e19
    x[5, 7] = 3e4
    return x


@pytest.mark.parametrize("mode", [0, 1])
@pytest.mark.parametrize("M,H", [(1, 3072), (200, 5376), (1000, 3072), (4100, 5376), (37, 8192), (300, 1000),
                                 (77, 520), (9, 8)])
def test_rms_quant(cuda, M, H, mode):
    from h3_tp2_amd import ops
    x, w, sh, sc, _, idx = mod_inputs(M, H, seed=M + H)
    x = _directed(x)
    ph = torch.full((M, H), float("nan"), dtype=BF16, device=cuda) if mode else None
    q, s = ops.rms_quant(x.to(cuda), w.to(cuda), *_tables(cuda, sh, sc), idx.to(cuda), EPS, ph)
    torch.cuda.synchronize()
    h_ref, q_ref, s_ref = O.rms_quant(bits16(x), bits16(w), bits16(sh), bits16(sc), idx.numpy(), EPS)
    assert q.shape == (M, H) and s.shape == (M, 1)
    assert_quant_equal(q, s, q_ref, s_ref)
    if mode:
        _nan_aware_equal(bits16(ph), h_ref, "h")


@pytest.mark.parametrize("mode", [0, 1])
@pytest.mark.parametrize("M,H", [(1, 3072), (200, 5376), (1000, 3072), (4100, 5376), (37, 8192), (300, 1000),
                                 (9, 8)])
def test_gate_rms_quant(cuda, M, H, mode):
    from h3_tp2_amd import ops
    x, w, sh, sc, gt, idx = mod_inputs(M, H, seed=M + H + 1)
    x = _directed(x)
    br = (torch.randn(M, H, generator=torch.Generator().manual_seed(M)) * 3).to(BF16)
    ph = torch.full((M, H), float("nan"), dtype=BF16, device=cuda) if mode else None
    gd, shd, scd = _tables(cuda, gt, sh, sc)
    res, q, s = ops.gate_rms_quant(x.to(cuda), gd, br.to(cuda), w.to(cuda), shd, scd, idx.to(cuda), EPS, ph)
    torch.cuda.synchronize()
    r_ref, h_ref, q_ref, s_ref = O.gate_rms_quant(bits16(x), bits16(gt), bits16(br), bits16(w), bits16(sh),
                                                  bits16(sc), idx.numpy(), EPS)
    _nan_aware_equal(bits16(res), r_ref, "residual_out")
    assert_quant_equal(q, s, q_ref, s_ref)
    if mode:
        _nan_aware_equal(bits16(ph), h_ref, "h")


def _order_rows(H: int, M: int = 256):
    """Rows whose fp32 variance depends on the order of the fp64 sum of squares: a pair 4096, 1 (squares summing to
    2^24 + 1, a tie between two fp32 values) and small elements +-2^-15 (square 2^-30, below half an fp64 ulp of
    2^24).  A small square added after the pair vanishes; small squares summed among themselves first survive once their
    sum passes half an fp64 ulp of 2^24, and a survivor makes the sum round to 2^24 + 2 instead of 2^24.  Rows of the first half have small
    elements everywhere: a sequential sum with the pair first gives 2^24, the fixed order (lane partials over chunks
    l, l + 64, ..., elements in order, then the xor butterfly) 2^24 + 2.  Rows of the second half have small elements
    only in the pair's own lane, so the result says how many of them precede the pair in that lane's partial (three or
    more survive it: 2^24 + 2).  Both are checked here on the CPU.  Returns x (bf16 [M, H]) and index runs
    (the workgroups of the staged forms take their LDS tables)."""
    g = torch.Generator().manual_seed(H)
    cpl = H // 512
    xf = torch.where(torch.rand(M, H, generator=g) < 0.5, -1.0, 1.0) * 2.0 ** -15
    lane = torch.randint(0, 64, (M,), generator=g)
    j = torch.randint(0, cpl, (M,), generator=g)
    j[M // 2::2] = 0                                   # half the pairs sit in their lane's first chunk
    pos = torch.randint(0, 7, (M,), generator=g)
    col = 8 * (lane + 64 * j) + pos
    keep = ((torch.arange(H) // 8) % 64)[None, :] == lane[M // 2:, None]     # second half: the pair's lane only
    xf[M // 2:] = torch.where(keep, xf[M // 2:], torch.zeros(()))
    rows = torch.arange(M)
    xf[rows, col] = 4096.0
    xf[rows, col + 1] = 1.0
    x = xf.to(BF16)
    assert torch.equal(x.float(), xf) and H % 512 == 0
    idx = torch.zeros(M, dtype=torch.int64)
    idx[M // 2:] = 1
    xb = bits16(x)
    sq = (x.float() * x.float()).double().numpy()

    def pair_first(m):                                 # the pair, then the small squares one by one: they vanish
        c = int(col[m])
        return np.float32(sum(np.concatenate([sq[m, c:c + 2], np.delete(sq[m], [c, c + 1])]).tolist()))
    fixed = np.array([np.float32(O.row_sumsq(xb[m])) for m in range(M)])
    low, high = np.float32(2.0 ** 24), np.float32(2.0 ** 24 + 2)
    assert all(pair_first(m) == low for m in range(M // 2)) and (fixed[:M // 2] == high).all()
    # k small squares ahead of the pair in its lane's partial: their sum k 2^-30 survives the pair's 2^24 once it is
    # past half an fp64 ulp there (2^-29, a tie that rounds to even for k = 2), so k >= 3 rounds up
    ahead = (8 * j + pos).numpy()[M // 2:]
    assert (ahead < 3).any() and (ahead >= 3).any()
    assert (fixed[M // 2:] == np.where(ahead >= 3, high, low)).all(), "the oracle's order is not the one stated"
    return x, idx


@pytest.mark.parametrize("H", [2048, 3072, 4096])
def test_rms_quant_order_sensitive_sums(cuda, H):
    """The qkv-site form (staged tables, 4 to 8 chunks per lane, reductions on register lane moves) on rows whose fp32
    variance depends on the summation order (_order_rows): the oracle's bits for fp8 bytes, scales and the bf16 row."""
    from h3_tp2_amd import ops
    x, idx = _order_rows(H)
    M = x.shape[0]
    _, w, sh, sc, _, _ = mod_inputs(M, H, seed=H + 7)
    ph = torch.full((M, H), float("nan"), dtype=BF16, device=cuda)
    q, s = ops.rms_quant(x.to(cuda), w.to(cuda), *_tables(cuda, sh, sc), idx.to(cuda), EPS, ph)
    torch.cuda.synchronize()
    h_ref, q_ref, s_ref = O.rms_quant(bits16(x), bits16(w), bits16(sh), bits16(sc), idx.numpy(), EPS)
    assert_quant_equal(q, s, q_ref, s_ref)
    _nan_aware_equal(bits16(ph), h_ref, "h")


@pytest.mark.parametrize("H", [2048, 3072, 4096])
@pytest.mark.parametrize("form", ["gate_rms_quant", "scale_gate_rms_quant"])
def test_gated_forms_order_sensitive_sums(cuda, H, form):
    """The gated forms on the same rows, the branch zero so that u = the residual: the fc1 producer (register form,
    LDS-permute butterfly) and the out consumer reading a zero fp32 product (staged tables, lane moves)."""
    from h3_tp2_amd import ops
    x, idx = _order_rows(H)
    M = x.shape[0]
    _, w, sh, sc, gt, _ = mod_inputs(M, H, seed=H + 8)
    gd, shd, scd = _tables(cuda, gt, sh, sc)
    br = torch.zeros(M, H, dtype=BF16)
    if form == "gate_rms_quant":
        res, q, s = ops.gate_rms_quant(x.to(cuda), gd, br.to(cuda), w.to(cuda), shd, scd, idx.to(cuda), EPS)
    else:
        x32 = torch.zeros(M, H, device=cuda)
        sa, sb = torch.full((M,), 0.5, device=cuda), torch.full((H,), 0.25, device=cuda)
        res, q, s = ops.scale_gate_rms_quant(x32, sa, sb, None, x.to(cuda), gd, w.to(cuda), shd, scd, idx.to(cuda),
                                             EPS, quant=True, modulated=False)
    torch.cuda.synchronize()
    r_ref, _, q_ref, s_ref = O.gate_rms_quant(bits16(x), bits16(gt), bits16(br), bits16(w), bits16(sh), bits16(sc),
                                              idx.numpy(), EPS)
    _nan_aware_equal(bits16(res), r_ref, "residual_out")
    assert_quant_equal(q, s, q_ref, s_ref)


def test_index_forms_and_strided_rows(cuda):
    """int32 indices, a strided index vector, x rows with a stride past H."""
    from h3_tp2_amd import ops
    M, H = 300, 3072
    x, w, sh, sc, gt, idx = mod_inputs(M, H, seed=11, B=9)
    xpad = torch.zeros(M, H + 64, dtype=BF16)
    xpad[:, :H] = x
    idx2 = torch.stack([idx, torch.zeros_like(idx)], dim=1).reshape(-1)[::2]      # stride 2
    assert idx2.stride(0) == 2
    h_ref, q_ref, s_ref = O.rms_quant(bits16(x), bits16(w), bits16(sh), bits16(sc), idx.numpy(), EPS)
    for ind in (idx.to(torch.int32).to(cuda), idx2.to(cuda)):
        q, s = ops.rms_quant(xpad.to(cuda)[:, :H], w.to(cuda), *_tables(cuda, sh, sc), ind, EPS)
        torch.cuda.synchronize()
        assert_quant_equal(q, s, q_ref, s_ref)


def test_index_out_of_range_poisons_only_its_row(cuda):
    """An index past the tables is not read through: that row's outputs are NaN, the other rows are unchanged."""
    from h3_tp2_amd import ops
    M, H = 16, 1024
    x, w, sh, sc, gt, idx = mod_inputs(M, H, seed=12, B=4)
    bad = idx.clone()
    bad[5] = 4
    bad[9] = -1
    br = (torch.randn(M, H, generator=torch.Generator().manual_seed(3))).to(BF16)
    ph = torch.empty((M, H), dtype=BF16, device=cuda)
    res, q, s = ops.gate_rms_quant(x.to(cuda), gt.to(cuda), br.to(cuda), w.to(cuda), sh.to(cuda), sc.to(cuda),
                                   bad.to(cuda), EPS, ph)
    torch.cuda.synchronize()
    ok = [m for m in range(M) if m not in (5, 9)]
    r_ref, h_ref, q_ref, s_ref = O.gate_rms_quant(bits16(x[ok]), bits16(gt), bits16(br[ok]), bits16(w), bits16(sh),
                                                  bits16(sc), idx[ok].numpy(), EPS)
    assert np.array_equal(bits16(res)[ok], r_ref) and np.array_equal(bits16(ph)[ok], h_ref)
    qb, sf = q.view(torch.uint8).cpu(), s.cpu()
    assert_quant_equal(qb[ok], sf[ok], q_ref, s_ref)
    for m in (5, 9):
        assert ((bits16(res)[m] & 0x7FFF) > 0x7F80).all() and ((bits16(ph)[m] & 0x7FFF) > 0x7F80).all()
        assert torch.isnan(sf[m]).item() and ((qb[m] & 0x7F) == 0x7F).all()


@pytest.mark.parametrize("M,H", [(1003, 3072), (61, 4096), (130, 2048), (45, 2560), (77, 1536), (29, 3000)])
def test_rms_quant_index_runs(cuda, M, H):
    """The qkv-site producer over index runs (one index per sample, as the model calls it): the 8-row workgroups whose
    rows share their first row's index read the tables staged in LDS, the workgroups that straddle a run boundary
    read the other rows' tables from global memory.  Runs of 1, 3, 5, 8, 13 and long ones, an index outside the tables
    at a workgroup's first row and inside one; every other row bit-exact against the oracle, h included."""
    from h3_tp2_amd import ops
    x, w, sh, sc, _, _ = mod_inputs(M, H, seed=M * 7 + H, B=5)
    x = _directed(x)
    runs = [1, 3, 5, 8, 13, 2, 40, 7, 9, 100]
    vals, k = [], 0
    while len(vals) < M:
        vals += [k % 5] * runs[k % len(runs)]
        k += 1
    idx = torch.tensor(vals[:M], dtype=torch.int64)
    bad = idx.clone()
    poisoned = [m for m in (16, 21) if m < M]
    for m in poisoned:
        bad[m] = 5 if m == 16 else -3
    ph = torch.full((M, H), float("nan"), dtype=BF16, device=cuda)
    q, s = ops.rms_quant(x.to(cuda), w.to(cuda), *_tables(cuda, sh, sc), bad.to(cuda), EPS, ph)
    torch.cuda.synchronize()
    ok = [m for m in range(M) if m not in poisoned]
    h_ref, q_ref, s_ref = O.rms_quant(bits16(x[ok]), bits16(w), bits16(sh), bits16(sc), idx[ok].numpy(), EPS)
    qb, sf = q.view(torch.uint8).cpu(), s.cpu()
    assert_quant_equal(qb[ok], sf[ok], q_ref, s_ref)
    _nan_aware_equal(bits16(ph)[ok], h_ref, "h")
    for m in poisoned:
        assert ((bits16(ph)[m] & 0x7FFF) > 0x7F80).all()
        assert torch.isnan(sf[m]).item() and ((qb[m] & 0x7F) == 0x7F).all()


def test_argument_errors(cuda):
    from h3_tp2_amd import _lib, ops
    x, w, sh, sc, _, idx = mod_inputs(4, 1004, seed=13)                   # H % 8 != 0
    with pytest.raises(_lib.H3Fp8Error, match="multiple of 8"):
        ops.rms_quant(x.to(cuda), w.to(cuda), sh.to(cuda), sc.to(cuda), idx.to(cuda), EPS)
    x, w, sh, sc, _, idx = mod_inputs(4, 64, seed=13)
    with pytest.raises(ValueError, match="indices"):
        ops.rms_quant(x.to(cuda), w.to(cuda), sh.to(cuda), sc.to(cuda), idx.float().to(cuda), EPS)
    q, s = ops.rms_quant(x[:0].to(cuda), w.to(cuda), sh.to(cuda), sc.to(cuda), idx[:0].to(cuda), EPS)
    assert q.shape == (0, 64) and s.shape == (0, 1)


def test_block_sites_end_to_end(cuda, monkeypatch):
    """The qkv and fc1 sites wired on a stand-in DiT block, on the GPU, with own_producers (the stock producers are
    the kernels' h-only form, so the fused form passes its self-check) and kernel 1 as the layers' quant: the QKV and
    fc1 layers receive the oracle's fp8 rows and scales, the block returns the oracle's residual_out."""
    import threading

    from _fake_dit import FakeQuantFP8, make_tr
    from _util import standin_gate_rms, standin_rms
    from h3_tp2_amd import fp8_quant_fuse as fq, ops

    st = dict(fq._state)
    st["checked"], st["disabled"] = {}, set()
    monkeypatch.setattr(fq, "_state", st)
    monkeypatch.setattr(fq, "_stats", dict.fromkeys(fq._stats, 0))
    monkeypatch.setattr(fq, "_tls", threading.local())
    monkeypatch.setattr(FakeQuantFP8, "forward", FakeQuantFP8.forward)
    monkeypatch.setattr(FakeQuantFP8, "impl", staticmethod(ops.quant_rows))
    tr = make_tr(standin_rms, standin_gate_rms)
    assert fq.install(("qkv", "fc1"), kernel1=False, tr=tr, quant_cls=FakeQuantFP8, lora_types=(),
                      own_producers=True, check_source=False) == ["qkv", "fc1"]
    M, H = 1000, 3072
    x, w, sh, sc, gt, idx = mod_inputs(M, H, seed=21)
    br = (torch.randn(M, H, generator=torch.Generator().manual_seed(22)) * 3).to(BF16)
    w2 = (w.float() * 0.75).to(BF16)
    gd, shd, scd = _tables(cuda, gt, sh, sc)
    blk = tr.MiniMaxH3DiTBlock(H, w.to(cuda), w2.to(cuda))
    res = blk(x.to(cuda), br.to(cuda), shd, scd, gd, idx.to(cuda))
    torch.cuda.synchronize()
    s = fq.stats()
    assert (s["fused_qkv"], s["fused_fc1"], s["consumed"], s["materialize"], s["selfcheck_fail"]) == (1, 1, 2, 0, 0)
    _, q_ref, s_ref = O.rms_quant(bits16(x), bits16(w), bits16(sh), bits16(sc), idx.numpy(), EPS)
    assert_quant_equal(*blk.attn.qkv_proj.seen[0], q_ref, s_ref)
    r_ref, _, q2_ref, s2_ref = O.gate_rms_quant(bits16(x), bits16(gt), bits16(br), bits16(w2), bits16(sh),
                                                bits16(sc), idx.numpy(), EPS)
    assert_quant_equal(*blk.mlp.fc1.seen[0], q2_ref, s2_ref)
    assert np.array_equal(bits16(res), r_ref)


def test_h_only_form_matches_the_fused_rows(cuda):
    """The producers without the quant (the own-producer form) give the fused form's bf16 rows bit for bit."""
    from h3_tp2_amd import ops
    M, H = 777, 5376
    x, w, sh, sc, gt, idx = mod_inputs(M, H, seed=23)
    br = (torch.randn(M, H, generator=torch.Generator().manual_seed(24))).to(BF16)
    shd, scd, gd = _tables(cuda, sh, sc, gt)
    h = ops.rms_norm_indexed_scale_shift(x.to(cuda), w.to(cuda), shd, scd, idx.to(cuda), EPS)
    res, h2 = ops.indexed_gate_rms_norm_scale_shift(x.to(cuda), gd, br.to(cuda), w.to(cuda), shd, scd, idx.to(cuda),
                                                    EPS)
    torch.cuda.synchronize()
    h_ref, _, _ = O.rms_quant(bits16(x), bits16(w), bits16(sh), bits16(sc), idx.numpy(), EPS)
    r_ref, h2_ref, _, _ = O.gate_rms_quant(bits16(x), bits16(gt), bits16(br), bits16(w), bits16(sh), bits16(sc),
                                           idx.numpy(), EPS)
    assert np.array_equal(bits16(h), h_ref)
    assert np.array_equal(bits16(res), r_ref) and np.array_equal(bits16(h2), h2_ref)


@pytest.mark.parametrize("gate,name", [(False, "c2_qkv_960x576_5s"), (True, "c3_ffn_1344x768_5s")])
def test_full_size_producers(cuda, gate, name):
    """The producers at the benchmark's full token counts (16740 and 31248 rows of 3072), against the oracle."""
    from h3_tp2_amd import ops, synthetic
    M, H = synthetic.CONFIGS[name]["M"], synthetic.CONFIGS[name]["K"]
    x, w, sh, sc, gt, idx = mod_inputs(M, H, seed=M)
    shd, scd, gd = _tables(cuda, sh, sc, gt)
    if gate:
        br = (torch.randn(M, H, generator=torch.Generator().manual_seed(5)) * 2).to(BF16)
        res, q, s = ops.gate_rms_quant(x.to(cuda), gd, br.to(cuda), w.to(cuda), shd, scd, idx.to(cuda), EPS)
        torch.cuda.synchronize()
        r_ref, _, q_ref, s_ref = O.gate_rms_quant(bits16(x), bits16(gt), bits16(br), bits16(w), bits16(sh),
                                                  bits16(sc), idx.numpy(), EPS)
        _nan_aware_equal(bits16(res), r_ref, "residual_out")
    else:
        q, s = ops.rms_quant(x.to(cuda), w.to(cuda), shd, scd, idx.to(cuda), EPS)
        torch.cuda.synchronize()
        _, q_ref, s_ref = O.rms_quant(bits16(x), bits16(w), bits16(sh), bits16(sc), idx.numpy(), EPS)
    assert_quant_equal(q, s, q_ref, s_ref)
