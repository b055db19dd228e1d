"""Source-fingerprint drift guards of the hook sites (CPU): a site is wired only when the upstream functions it relies
on fingerprint to the reviewed sources; a changed, missing or foreign-wrapped function leaves it stock with a warning
naming the function.  Stand-in transformer and upstream modules here; the reviewed table is made from them."""
import functools
import types

import pytest
import torch

from h3_tp2_amd import _drift, _sites, fp8_consumers, fp8_gemm, fp8_swiglu


def test_fingerprint_normalisation():
    base = "def f(x):\n    return x + 1\n"
    # known answer: sha256 of the stripped lines "def f(x):" and "return x + 1" joined by a newline, 16 hex digits
    assert _drift.fingerprint_source(base) == "5ef880d55750a5d2"
    noisy = "@decorator\ndef f(x):\n\n    # a comment\n        return x + 1   \n"
    assert _drift.fingerprint_source(noisy) == "5ef880d55750a5d2"
    assert _drift.fingerprint_source("def f(x):\n    return x + 2\n") != "5ef880d55750a5d2"


# ---- stand-in upstream -------------------------------------------------------------------------------------------

def _block_forward(self, x):
    return x


def _attn_forward(self, x):
    return x


def _mlp_forward(self, x):
    h, _ = self.fc1(x)
    return self.fc2(self.act_fn(h))[0]


def _kernel(*args):
    return None


def _launcher(*args):
    return None


def _indexed_gate(x, gate, other, indices):
    return x


def _gate_rms(residual, gate, branch, weight, shift, scale, indices, eps):
    return residual, branch


def _rms(x, weight, shift, scale, indices, eps):
    return x


def _qk(q, k, q_weight, k_weight, rope, eps):
    return q, k


def _fake_upstream():
    tr = types.ModuleType("fake_transformer")
    tr.MiniMaxH3DiTBlock = type("MiniMaxH3DiTBlock", (), {"forward": _block_forward})
    tr.MiniMaxH3Attention = type("MiniMaxH3Attention", (), {"forward": _attn_forward})
    tr.MiniMaxH3MLP = type("MiniMaxH3MLP", (torch.nn.Module,), {"forward": _mlp_forward})
    tr.fused_qk_norm_rope, tr.indexed_gate = _qk, _indexed_gate
    tr.indexed_gate_rms_norm_scale_shift, tr.rms_norm_indexed_scale_shift = _gate_rms, _rms
    qk = types.SimpleNamespace(_rms_norm_rope_kernel=_kernel, _launch_fused_rms_norm_rope=_launcher,
                               _fused_qk_norm_rope_impl=_launcher, _fused_cuda_supported=_launcher,
                               fused_qk_norm_rope=_qk)
    im = types.SimpleNamespace(_indexed_gate_kernel=_kernel, _indexed_gate_rms_norm_scale_shift_kernel=_kernel,
                               _rms_norm_indexed_scale_shift_kernel=_kernel, _launch_row_chunks=_launcher,
                               indexed_gate=_indexed_gate, indexed_gate_rms_norm_scale_shift=_gate_rms,
                               rms_norm_indexed_scale_shift=_rms)
    act = types.SimpleNamespace(SiluAndMul=type("SiluAndMul", (), {"forward_cuda": _launcher}))
    linear = types.SimpleNamespace(ColumnParallelLinear=type("C", (), {"forward": _launcher}),
                                   RowParallelLinear=type("R", (), {"forward": _launcher}))
    smm = types.SimpleNamespace(FP8ScaledMMLinearKernel=type("K", (), {"apply_weights": _launcher}))
    modules = {"qk": qk, "im": im, "act": act, "linear": linear, "smm": smm}
    found = _drift.resolvers(tr, modules)
    reviewed = {name: _drift.fingerprint(get()) for name, get in found.items() if get() is not None}
    return tr, modules, reviewed


@pytest.fixture
def notes(caplog):
    caplog.set_level("WARNING")
    return _sites.Notes(__import__("logging").getLogger("test_drift"), "")


def test_all_sites_kept_over_the_reviewed_sources(notes):
    tr, modules, reviewed = _fake_upstream()
    for protocol, sites in _drift.NEEDS.items():
        assert _drift.keep_sites(protocol, tuple(sites), tr, notes, reviewed, modules) == tuple(sites)


def test_a_changed_function_skips_exactly_the_sites_that_need_it(notes, caplog):
    tr, modules, reviewed = _fake_upstream()

    def _indexed_gate_v2(x, gate, other, indices):
        return x + 0
    tr.indexed_gate = modules["im"].indexed_gate = _indexed_gate_v2     # upstream changed fc2's consumer
    assert _drift.keep_sites("consumers", ("qkv", "out", "fc2"), tr, notes, reviewed, modules) == ("qkv", "out")
    assert "site fc2 skipped" in caplog.text and "indexed_gate:" in caplog.text

    def _block_forward_v2(self, x):
        return self.attn(x)
    tr.MiniMaxH3DiTBlock.forward = _block_forward_v2          # every site relies on the block forward
    assert _drift.keep_sites("producers", ("qkv", "fc1", "fc2"), tr, notes, reviewed, modules) == ()


def test_a_missing_function_skips_the_site(notes, caplog):
    tr, modules, reviewed = _fake_upstream()
    del modules["act"].SiluAndMul.forward_cuda
    assert _drift.keep_sites("producers", ("qkv", "fc1", "fc2"), tr, notes, reviewed, modules) == ("qkv", "fc1")
    assert "silu_forward_cuda: absent" in caplog.text
    del modules["im"]
    assert _drift.keep_sites("consumers", ("qkv", "out", "fc2"), tr, notes, reviewed, modules) == ("qkv",)


def test_method_wrappers_are_seen_through(notes):
    """As in the reference, a method's source is read through functools.wraps (inspect unwraps it)."""
    tr, modules, reviewed = _fake_upstream()
    tr.MiniMaxH3DiTBlock.forward = functools.wraps(_block_forward)(lambda self, x: _block_forward(self, x))
    assert _drift.keep_sites("consumers", ("qkv",), tr, notes, reviewed, modules) == ("qkv",)


@pytest.mark.parametrize("with_wraps", [False, True])
def test_a_foreign_wrapper_of_a_by_name_binding_is_drift(notes, caplog, with_wraps):
    """The transformer must call the upstream function itself (h3_tp2/fp8_consumers.py:849-855): a wrapper someone
    else put there -- even one made with functools.wraps, whose source reads as the upstream function's -- leaves the
    site stock, since the fused consumer would replace the call and drop the wrapper's behaviour."""
    tr, modules, reviewed = _fake_upstream()

    def foreign(x, gate, other, indices):
        return _indexed_gate(x, gate, other, indices)
    tr.indexed_gate = functools.wraps(_indexed_gate)(foreign) if with_wraps else foreign
    assert _drift.keep_sites("consumers", ("qkv", "fc2"), tr, notes, reviewed, modules) == ("qkv",)
    assert "indexed_gate: wrapped" in caplog.text


def test_this_librarys_own_wrappers_are_seen_through(notes):
    """A binding that is this library's wrapper of the upstream function (code in this package, an _h3_tp2_amd*
    marker, __wrapped__) is accepted, also nested; the same marker copied onto a foreign wrapper by functools.wraps is
    not enough (its code lives elsewhere)."""
    tr, modules, reviewed = _fake_upstream()
    own = fp8_consumers.make_consumer_wrapper("fc2", _indexed_gate)
    assert _drift.is_own_wrapper(own) and own.__wrapped__ is _indexed_gate
    tr.indexed_gate = own
    assert _drift.keep_sites("consumers", ("fc2",), tr, notes, reviewed, modules) == ("fc2",)
    tr.indexed_gate = fp8_consumers.make_consumer_wrapper("fc2", own)
    assert _drift.keep_sites("consumers", ("fc2",), tr, notes, reviewed, modules) == ("fc2",)

    def foreign(*args):
        return own(*args)
    foreign = functools.wraps(own)(foreign)                  # copies own's marker and sets __wrapped__ = own
    assert not _drift.is_own_wrapper(foreign)
    tr.indexed_gate = foreign
    assert _drift.keep_sites("consumers", ("fc2",), tr, notes, reviewed, modules) == ()


def test_consumer_install_skips_drifted_sites(monkeypatch):
    monkeypatch.setitem(fp8_gemm._state, "level", "tensor32")
    monkeypatch.setitem(fp8_gemm._state, "fused", False)
    monkeypatch.setattr(fp8_consumers, "_state", {"sites": (), "disabled": set(), "fused": {}, "checked": {}})
    tr, modules, reviewed = _fake_upstream()
    reviewed = dict(reviewed, gate_rms_kernel="0000000000000000")        # the out site's kernel was not reviewed
    try:
        assert fp8_consumers.install(("qkv", "out", "fc2"), tr=tr, lora_types=(), reviewed=reviewed,
                                     modules=modules) == ["qkv", "fc2"]
        assert not getattr(tr.indexed_gate_rms_norm_scale_shift, "_h3_tp2_amd_consumer", False)   # out stays stock
        assert tr.indexed_gate._h3_tp2_amd_consumer and tr.fused_qk_norm_rope._h3_tp2_amd_consumer
    finally:
        fp8_gemm.clear_hooks()


def test_swiglu_install_checks_the_mlp_forward(monkeypatch):
    monkeypatch.setattr(fp8_swiglu, "_state", dict(fp8_swiglu._state))
    tr, modules, reviewed = _fake_upstream()
    try:
        assert not fp8_swiglu.install(1, tr=tr, check=False, reviewed=dict(reviewed, mlp_forward="0" * 16))
        assert tr.MiniMaxH3MLP.forward is _mlp_forward
        assert fp8_swiglu.install(1, tr=tr, check=False, reviewed=reviewed)
        assert tr.MiniMaxH3MLP.forward is not _mlp_forward
        # the wrapped forward still fingerprints as the upstream one
        assert _drift.fingerprint(tr.MiniMaxH3MLP.forward) == reviewed["mlp_forward"]
    finally:
        fp8_gemm.clear_hooks()


def test_consumer_install_leaves_router_sites_stock(monkeypatch, caplog):
    """With the block router registered (the two-pass level plus kernel 2 for the block's qkv / out / fc1, the
    reference's cutlass layout), qkv and out are computed in bf16 ahead of the stash hook: their consumers stay stock
    and only fc2 is fused (h3_tp2/fp8_consumers.py:870-877)."""
    monkeypatch.setitem(fp8_gemm._state, "level", "tensor32")
    monkeypatch.setitem(fp8_gemm._state, "fused", False)
    monkeypatch.setattr(fp8_consumers, "_state", {"sites": (), "disabled": set(), "fused": {}, "checked": {}})
    tr, modules, reviewed = _fake_upstream()
    from h3_tp2_amd import fp8_hip
    caplog.set_level("WARNING")
    try:
        fp8_gemm.set_router(fp8_hip.route)
        assert fp8_consumers.install(("qkv", "out", "fc2"), tr=tr, lora_types=(), reviewed=reviewed,
                                     modules=modules) == ["fc2"]
        assert tr.fused_qk_norm_rope is _qk and tr.indexed_gate_rms_norm_scale_shift is _gate_rms
        assert tr.indexed_gate._h3_tp2_amd_consumer
        assert "block router computes qkv, out" in caplog.text
    finally:
        fp8_gemm.clear_hooks()
