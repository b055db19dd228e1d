"""CPU tests of the qkv / fc1 producer sites (the RMS-norm + AdaLN producers with the quant fused in): routing,
the two-mode self-check, disabling, the reload mode, materialisation and install rules, on a stand-in DiT block with
CPU mirrors in place of the kernels.  Mirrors what the reference's tests/test_fp8_quant_fuse.py:150-200 checks
(site subsets, a self-check mismatch disables the site, mode 0 failing falls back to mode 1)."""
import threading

import numpy as np

import pytest
import torch

from _fake_dit import FakeQuantFP8, make_tr
from _util import mod_inputs, standin_gate_rms, standin_rms
from h3_tp2_amd import fp8_quant_fuse as fq

E4M3 = torch.float8_e4m3fn
BF16 = torch.bfloat16
H = 256


def torch_quant(h):
    """The per-token quant formula in torch (CPU): both the stock quant and the mirrors' quant here."""
    hf = h.float()
    s = torch.clamp(hf.abs().amax(dim=1, keepdim=True) / 448.0, min=fq.MIN_SCALE)
    return (hf * (1.0 / s)).clamp(-448.0, 448.0).to(E4M3), s


def mirror_rms_quant(x, weight, shift, scale, indices, eps, stock=None, ph=None):
    h = standin_rms(x, weight, shift, scale, indices, eps)
    if ph is not None:
        ph.copy_(h)
    return torch_quant(h)


def mirror_gate_rms_quant(residual, gate, branch, weight, shift, scale, indices, eps, stock=None, ph=None):
    res, h = standin_gate_rms(residual, gate, branch, weight, shift, scale, indices, eps)
    if ph is not None:
        ph.copy_(h)
    return (res, *torch_quant(h))


@pytest.fixture
def fuse(monkeypatch):
    st = dict(fq._state)
    st["checked"], st["disabled"] = {}, set()
    monkeypatch.setattr(fq, "_state", st)
    monkeypatch.setattr(fq, "_stats", dict.fromkeys(fq._stats, 0))
    monkeypatch.setattr(fq, "_tls", threading.local())
    monkeypatch.setattr(fq, "_warned", set())
    monkeypatch.setattr(FakeQuantFP8, "forward", FakeQuantFP8.forward)       # restored after install wraps it
    monkeypatch.setattr(FakeQuantFP8, "impl", staticmethod(torch_quant))
    monkeypatch.setattr(fq, "producer_takes", lambda *a: True)
    monkeypatch.setattr(fq, "rms_quant", mirror_rms_quant)
    monkeypatch.setattr(fq, "gate_rms_quant", mirror_gate_rms_quant)
    return fq


def _inputs(M=96):
    x, w, sh, sc, gt, idx = mod_inputs(M, H, seed=M)
    br = (torch.randn(M, H, generator=torch.Generator().manual_seed(1)) * 2).to(BF16)
    w2 = (w.float() * 1.5).to(BF16)
    return x, br, sh, sc, gt, idx, w, w2


def _run(tr, inp):
    x, br, sh, sc, gt, idx, w, w2 = inp
    blk = tr.MiniMaxH3DiTBlock(H, w, w2)
    res = blk(x, br, sh, sc, gt, idx)
    return blk, res


def _same(a, b):
    (qa, sa), (qb, sb) = a, b
    return torch.equal(qa.view(torch.uint8), qb.view(torch.uint8)) and torch.equal(sa, sb)


def _reference(inp):
    tr = make_tr(standin_rms, standin_gate_rms)
    return _run(tr, inp)


def _install(fuse, tr, sites=("qkv", "fc1"), **kw):
    """The sites over the stand-in stock producers; the fused mirrors here share the stand-ins' arithmetic, so the
    caller vouches for the self-check (the default leaves the reducing sites stock: test_default_install_...)."""
    kw.setdefault("trust_selfcheck", True)
    kw.setdefault("check_source", False)         # the stand-in module is not the reviewed upstream
    return fuse.install(sites, kernel1=False, tr=tr, quant_cls=FakeQuantFP8, lora_types=(), **kw)


def test_sites_fused_and_equal_to_stock(fuse):
    inp = _inputs()
    ref_blk, ref_res = _reference(inp)
    tr = make_tr(standin_rms, standin_gate_rms)
    assert _install(fuse, tr) == ["qkv", "fc1"]
    blk, res = _run(tr, inp)
    assert torch.equal(res, ref_res)
    assert _same(blk.attn.qkv_proj.seen[0], ref_blk.attn.qkv_proj.seen[0])
    assert _same(blk.mlp.fc1.seen[0], ref_blk.mlp.fc1.seen[0])
    s = fuse.stats()
    assert (s["fused_qkv"], s["fused_fc1"], s["consumed"], s["materialize"]) == (1, 1, 2, 0)
    assert s["selfcheck_pass"] == 2 and s["selfcheck_fail"] == 0           # mode 0 passes at both sites
    _run(tr, inp)
    assert fuse.stats()["selfcheck_pass"] == 2 and fuse.stats()["fused_qkv"] == 2   # checked once per key


@pytest.mark.parametrize("sites", [("qkv",), ("fc1",)])
def test_site_subsets(fuse, sites):
    inp = _inputs()
    ref_blk, ref_res = _reference(inp)
    tr = make_tr(standin_rms, standin_gate_rms)
    assert _install(fuse, tr, sites) == list(sites)
    blk, res = _run(tr, inp)
    assert torch.equal(res, ref_res) and _same(blk.mlp.fc1.seen[0], ref_blk.mlp.fc1.seen[0])
    s = fuse.stats()
    assert s["consumed"] == 1 and all(s["fused_" + x] == (x in sites) for x in ("qkv", "fc1"))


def test_selfcheck_mismatch_disables_site(fuse, monkeypatch):
    inp = _inputs()
    ref_blk, ref_res = _reference(inp)

    def off_by_one(*a, **k):
        q, s = mirror_rms_quant(*a, **k)
        q = q.clone()
        q.view(torch.uint8)[0, 3] ^= 1
        return q, s
    monkeypatch.setattr(fq, "rms_quant", off_by_one)
    tr = make_tr(standin_rms, standin_gate_rms)
    _install(fuse, tr)
    blk, res = _run(tr, inp)
    assert torch.equal(res, ref_res) and _same(blk.attn.qkv_proj.seen[0], ref_blk.attn.qkv_proj.seen[0])
    s = fuse.stats()
    assert s["selfcheck_fail"] == 2 and s["fused_qkv"] == 0 and "qkv" in fq._state["disabled"]   # both modes tried
    assert s["fused_fc1"] == 1
    _run(tr, inp)
    assert fuse.stats()["selfcheck_fail"] == 2                                 # disabled: not checked again


@pytest.mark.parametrize("site", ["qkv", "fc1"])
def test_reload_mode_when_registers_differ(fuse, monkeypatch, site):
    """Mode 0 (bf16 row only in registers) failing its self-check falls back to mode 1 (the bf16 row stored too)."""
    inp = _inputs()
    ref_blk, ref_res = _reference(inp)
    name = {"qkv": "rms_quant", "fc1": "gate_rms_quant"}[site]
    real = {"qkv": mirror_rms_quant, "fc1": mirror_gate_rms_quant}[site]
    modes = []

    def wrong_in_registers(*a, **k):
        out = real(*a, **k)
        ph = a[7 if site == "qkv" else 9]
        modes.append(ph is not None)
        if ph is None:
            q = out[-2].clone()
            q.view(torch.uint8)[0, 0] ^= 1
            out = (*out[:-2], q, out[-1])
        return out
    monkeypatch.setattr(fq, name, wrong_in_registers)
    tr = make_tr(standin_rms, standin_gate_rms)
    _install(fuse, tr)
    blk, res = _run(tr, inp)
    layer = blk.attn.qkv_proj if site == "qkv" else blk.mlp.fc1
    ref_layer = ref_blk.attn.qkv_proj if site == "qkv" else ref_blk.mlp.fc1
    assert torch.equal(res, ref_res) and _same(layer.seen[0], ref_layer.seen[0])
    assert modes == [False, True, True]        # mode 0 checked, mode 1 checked, mode 1 run on the whole tensor
    assert fuse.stats()["fused_" + site] == 1 and fuse.stats()["selfcheck_fail"] == 1


def test_foreign_weight_or_unplanned_call_stays_stock(fuse):
    """A producer call whose weight is not the block's norm weight, or outside a DiT block, runs the stock producer."""
    inp = _inputs()
    x, br, sh, sc, gt, idx, w, w2 = inp
    tr = make_tr(standin_rms, standin_gate_rms)
    _install(fuse, tr)
    h = tr.rms_norm_indexed_scale_shift(x, w, sh, sc, idx, 1e-6)                # no block context
    assert torch.equal(h, standin_rms(x, w, sh, sc, idx, 1e-6))

    class Other(tr.MiniMaxH3DiTBlock):
        def forward(self, x, branch, shift, scale, gate, idx):
            h = tr.rms_norm_indexed_scale_shift(x, w2, shift, scale, idx, 1e-6)   # not norm1.weight
            self.attn.qkv_proj(h)
            return h
    Other.forward = fq.make_block_forward(Other.forward, ("qkv", "fc1"), ())     # the block context, as installed
    blk = Other(H, w, w2)
    blk(x, br, sh, sc, gt, idx)
    assert fuse.stats()["fused_qkv"] == 0 and fuse.stats()["consumed"] == 0


def test_stash_not_consumed_is_materialised(fuse):
    """The QKV layer quantises another tensor than the placeholder: the stash is materialised (the stock producer into
    the placeholder) and the layer's quant runs on what it was given."""
    inp = _inputs()
    x, br, sh, sc, gt, idx, w, w2 = inp
    tr = make_tr(standin_rms, standin_gate_rms)
    _install(fuse, tr, ("qkv",))
    seen = {}

    class Copying(tr.MiniMaxH3DiTBlock):
        def forward(self, x, branch, shift, scale, gate, idx):
            h = tr.rms_norm_indexed_scale_shift(x, self.norm1.weight, shift, scale, idx, 1e-6)
            self.attn.qkv_proj(h.clone())
            seen["h"] = h
            return h
    Copying.forward = fq.make_block_forward(Copying.forward, ("qkv",), ())
    blk = Copying(H, w, w2)
    blk(x, br, sh, sc, gt, idx)
    s = fuse.stats()
    assert s["fused_qkv"] == 1 and s["materialize"] == 1 and s["consumed"] == 0
    assert torch.equal(seen["h"], standin_rms(x, w, sh, sc, idx, 1e-6))       # mode 0 placeholder filled by stock


def test_install_skips_fc1_when_the_consumer_hook_owns_it(fuse):
    tr = make_tr(standin_rms, standin_gate_rms)
    tr.indexed_gate_rms_norm_scale_shift._h3_tp2_amd_consumer = True
    try:
        assert _install(fuse, tr) == ["qkv"]
    finally:
        del standin_gate_rms._h3_tp2_amd_consumer


def test_install_out_site_is_skipped_and_idempotent(fuse):
    tr = make_tr(standin_rms, standin_gate_rms)
    assert _install(fuse, tr, ("qkv", "out")) == ["qkv"]
    wrapped = tr.rms_norm_indexed_scale_shift
    assert wrapped.__wrapped__ is standin_rms
    _install(fuse, tr, ("qkv",))
    assert tr.rms_norm_indexed_scale_shift is wrapped


def test_own_producers_sit_below_the_fused_wrappers(fuse, monkeypatch):
    """own_producers: the stock producers are replaced by the kernels' h-only form (here a recorder) and the fused
    wrappers call that form as their stock; inputs it does not take still reach the original."""
    calls = []
    monkeypatch.setattr(fq.ops, "rms_norm_indexed_scale_shift",
                        lambda *a: calls.append("rms") or standin_rms(*a))
    monkeypatch.setattr(fq.ops, "indexed_gate_rms_norm_scale_shift",
                        lambda *a: calls.append("gate") or standin_gate_rms(*a))
    tr = make_tr(standin_rms, standin_gate_rms)
    _install(fuse, tr, own_producers=True)
    own = tr.rms_norm_indexed_scale_shift.__wrapped__
    assert own._h3_tp2_amd_own and own.__wrapped__ is standin_rms
    inp = _inputs()
    ref_blk, ref_res = _reference(inp)
    blk, res = _run(tr, inp)
    assert torch.equal(res, ref_res) and calls.count("rms") == 1 and calls.count("gate") == 1   # the self-checks
    monkeypatch.setattr(fq, "producer_takes", lambda *a: False)
    x, br, sh, sc, gt, idx, w, w2 = inp
    own(x, w, sh, sc, idx, 1e-6)
    assert calls.count("rms") == 1


def test_producer_takes_rules():
    x, w, sh, sc, gt, idx = mod_inputs(8, 64, seed=2)
    assert not fq.producer_takes(x, w, (sh, sc), idx)                           # CPU tensors: never


def test_default_install_keeps_the_reducing_sites_stock(fuse, caplog):
    """Without own_producers and without the caller vouching for the stock reduction, the qkv / fc1 sites are not
    wired (a warning says so) and the block runs the stock producers; the fc2 site would still be wired."""
    tr = make_tr(standin_rms, standin_gate_rms)
    with caplog.at_level("WARNING"):
        assert fuse.install(("qkv", "fc1"), kernel1=False, tr=tr, quant_cls=FakeQuantFP8, lora_types=(),
                            check_source=False) == []
    assert "qkv stays stock" in caplog.text and "fc1 stays stock" in caplog.text
    assert tr.rms_norm_indexed_scale_shift is standin_rms and tr.indexed_gate_rms_norm_scale_shift is standin_gate_rms
    inp = _inputs()
    ref_blk, ref_res = _reference(inp)
    blk, res = _run(tr, inp)
    assert torch.equal(res, ref_res) and _same(blk.attn.qkv_proj.seen[0], ref_blk.attn.qkv_proj.seen[0])
    assert fuse.stats()["fused_qkv"] == 0 and fuse.stats()["selfcheck_pass"] == 0


def _fp64_sum_rms_quant(x, weight, shift, scale, indices, eps, stock=None, ph=None):
    """The producer kernel's arithmetic (squares summed in fp64, one rounding), through the oracle."""
    from oracle import oracle as O
    from _util import bits16
    h, q, sc = O.rms_quant(bits16(x), bits16(weight), bits16(shift), bits16(scale), indices.numpy(), eps)
    hb = torch.from_numpy(h.view("int16")).view(BF16)
    if ph is not None:
        ph.copy_(hb)
    return torch.from_numpy(q).view(E4M3), torch.from_numpy(sc).view(-1, 1)


def test_fp64_sum_against_the_fp32_standin_falls_back_cleanly(fuse, monkeypatch):
    """The reference's torch stand-in (fp32 sum) as the stock producer, the kernel's fp64-sum arithmetic as the fused
    one.  The two sums differ on about 40 % of the rows, the bf16 rows on about 1 % (a one-ulp move of the sum rarely
    crosses a bf16 rounding boundary) and the fp8 row the QKV GEMM reads on about 0.05 % (the bf16 move must also cross
    an e4m3 boundary).  With such a row among the self-check's sampled rows both modes fail, the qkv site is disabled
    and the block's results equal the stock path's."""
    from oracle import oracle as O
    from _util import bits16
    H1 = 1024
    xp, w, sh, sc, gt, idxp = mod_inputs(3000, H1, seed=5)         # rows 193, 1352, 1376, 1829 differ in fp8
    _, q_k, s_k = O.rms_quant(bits16(xp), bits16(w), bits16(sh), bits16(sc), idxp.numpy(), 1e-6)
    q_s, s_s = O.quant_rows(bits16(standin_rms(xp, w, sh, sc, idxp, 1e-6)))
    differ = np.nonzero((q_k != q_s).any(1) | (s_k.view(np.uint32) != s_s.view(np.uint32)))[0]
    assert differ.size, "the pool must hold a row whose fp8 bytes differ between the two sums"
    pick = torch.from_numpy(np.concatenate([differ[:1], np.setdiff1d(np.arange(96), differ[:1])[:95]]))
    x, idx = xp[pick].contiguous(), idxp[pick].contiguous()
    monkeypatch.setattr(fq, "rms_quant", _fp64_sum_rms_quant)
    tr = make_tr(standin_rms, standin_gate_rms)
    _install(fuse, tr, ("qkv",))
    br = torch.zeros(96, H1, dtype=BF16)
    blk = tr.MiniMaxH3DiTBlock(H1, w, w)
    res = blk(x, br, sh, sc, gt, idx)
    ref = make_tr(standin_rms, standin_gate_rms).MiniMaxH3DiTBlock(H1, w, w)
    ref_res = ref(x, br, sh, sc, gt, idx)
    assert torch.equal(res, ref_res) and _same(blk.attn.qkv_proj.seen[0], ref.attn.qkv_proj.seen[0])
    s = fuse.stats()
    assert s["fused_qkv"] == 0 and s["selfcheck_fail"] == 2 and "qkv" in fq._state["disabled"]


def test_fp64_sum_rows_outside_the_sample_are_why_the_default_is_stock(fuse, monkeypatch):
    """The same pair with the fp8-differing row past the 64 sampled rows: the self-check passes (mode 0: the sampled
    rows' fp8 bytes agree) and the site engages, so that row's fp8 bytes differ from the stock path's.  This is the
    case the default install avoids by keeping the reducing sites stock unless the producers are the library's own."""
    from oracle import oracle as O
    from _util import bits16
    H1 = 1024
    xp, w, sh, sc, gt, idxp = mod_inputs(3000, H1, seed=5)
    _, q_k, s_k = O.rms_quant(bits16(xp), bits16(w), bits16(sh), bits16(sc), idxp.numpy(), 1e-6)
    q_s, s_s = O.quant_rows(bits16(standin_rms(xp, w, sh, sc, idxp, 1e-6)))
    differ = np.nonzero((q_k != q_s).any(1) | (s_k.view(np.uint32) != s_s.view(np.uint32)))[0]
    same = np.setdiff1d(np.arange(200), differ)[:95]
    pick = torch.from_numpy(np.concatenate([same, differ[:1]]))          # the differing row last (row 95)
    x, idx = xp[pick].contiguous(), idxp[pick].contiguous()
    monkeypatch.setattr(fq, "rms_quant", _fp64_sum_rms_quant)
    tr = make_tr(standin_rms, standin_gate_rms)
    _install(fuse, tr, ("qkv",))
    br = torch.zeros(96, H1, dtype=BF16)
    blk = tr.MiniMaxH3DiTBlock(H1, w, w)
    blk(x, br, sh, sc, gt, idx)
    ref = make_tr(standin_rms, standin_gate_rms).MiniMaxH3DiTBlock(H1, w, w)
    ref(x, br, sh, sc, gt, idx)
    assert fuse.stats()["fused_qkv"] == 1
    (qa, sa), (qb, sb) = blk.attn.qkv_proj.seen[0], ref.attn.qkv_proj.seen[0]
    rows_differ = ((qa.view(torch.uint8) != qb.view(torch.uint8)).any(1) | (sa != sb).view(-1)).nonzero().view(-1)
    assert rows_differ.tolist() == [95]
