"""CPU tests of the host-side hook surface (dispatcher, router, SwiGLU stash, quant stash, consumer stash).

These check routing, eligibility and the stash protocols with stand-in compute (the kernels need the GPU; here the
launch functions are replaced by recorders).  Mirrors the reference's tests/test_fp8_cutlass_routing.py,
tests/test_fp8_gemm.py (dispatcher), tests/test_fp8_swiglu.py (stash hook) and tests/test_fp8_quant_fuse.py
(Pending protocol) in what they check.
"""
import threading

import pytest
import torch

from h3_tp2_amd import fp8_consumers, fp8_gemm, fp8_hip, fp8_quant_fuse, fp8_swiglu, ops

E4M3 = torch.float8_e4m3fn
BF16 = torch.bfloat16


@pytest.fixture(autouse=True)
def _clean(monkeypatch):
    fp8_gemm.clear_hooks()
    monkeypatch.setitem(fp8_gemm._state, "fused", True)
    monkeypatch.setitem(fp8_gemm._state, "level", "hip")
    yield
    fp8_gemm.clear_hooks()


class Recorder:
    def __init__(self, tag):
        self.tag, self.calls = tag, []

    def __call__(self, a, b, scale_a, scale_b, out_dtype, bias=None):
        self.calls.append((a, b, scale_a, scale_b, out_dtype, bias))
        return torch.full((a.shape[0], b.shape[1]), len(self.calls), dtype=out_dtype)


def operands(M=32, K=64, N=48):
    a = torch.zeros(M, K).to(E4M3)
    w = torch.zeros(N, K).to(E4M3)          # [N, K] row-major; vLLM passes b = w.t() [K, N]
    return a, w.t(), torch.ones(M, 1), torch.ones(N)


# ---- dispatcher -----------------------------------------------------------------------------------------------------

class FakeOps:
    def __init__(self):
        self.stock = Recorder("stock")
        self.cutlass_scaled_mm = self.stock


def test_eligibility_matches_reference_rules():
    a, b, sa, sb = operands()
    assert fp8_gemm.eligible(a, b, sa, sb, BF16)
    assert fp8_gemm.eligible(a, b, sa, sb, torch.float16)
    assert fp8_gemm.eligible(a, b, sa.view(-1), sb.view(1, -1), BF16)
    assert fp8_gemm.eligible(a, b, torch.ones(()), sb, BF16)               # scalar a-scale, vector b-scale
    assert fp8_gemm.eligible(a, b, sa, torch.ones(()), BF16, torch.zeros(48, dtype=BF16))
    assert not fp8_gemm.eligible(a, b, torch.ones(()), torch.ones(()), BF16)   # per-tensor: stock
    assert not fp8_gemm.eligible(a, b, torch.ones(16, 1), sb, BF16)        # block scales: stock
    assert not fp8_gemm.eligible(a, b, sa, torch.ones(24), BF16)
    assert not fp8_gemm.eligible(a, b, sa.double(), sb, BF16)
    assert not fp8_gemm.eligible(a.float(), b, sa, sb, BF16)
    assert not fp8_gemm.eligible(a, b, sa, sb, torch.float32)
    assert not fp8_gemm.eligible(a, b, sa, sb, BF16, torch.zeros(47, dtype=BF16))
    assert not fp8_gemm.eligible(a, b, sa, sb, BF16, torch.zeros(1, 48, dtype=BF16))
    assert not fp8_gemm.eligible(a.t().contiguous().t(), b, sa, sb, BF16)    # A not row-major
    assert not fp8_gemm.eligible(a, b.contiguous(), sa, sb, BF16)            # B^T not contiguous
    a2, b2, sa2, sb2 = operands(K=72)
    assert not fp8_gemm.eligible(a2, b2, sa2, sb2, BF16)                      # K % 16
    a3, b3, sa3, sb3 = operands(N=40)
    assert not fp8_gemm.eligible(a3, b3, sa3, sb3, BF16)                      # N % 16
    assert not fp8_gemm.eligible(a.unsqueeze(0), b, sa, sb, BF16)
    assert not fp8_gemm.eligible(a, operands(K=80)[1], sa, sb, BF16)          # K mismatch
    a4, b4, sa4, sb4 = operands(K=0)
    assert not fp8_gemm.eligible(a4, b4, sa4, sb4, BF16)                      # empty reduction


def test_install_routes_eligible_calls_and_keeps_stock(monkeypatch):
    fake = FakeOps()
    hip = Recorder("hip")
    monkeypatch.setattr(fp8_gemm, "scaled_mm_fused", hip)
    monkeypatch.setattr(fp8_gemm, "_state", dict(fp8_gemm._state))
    assert fp8_gemm.install(fake, level="hip", check=False)
    assert fake.cutlass_scaled_mm is not fake.stock and fake.cutlass_scaled_mm.__wrapped__ is fake.stock
    assert fp8_gemm._state["fused"] and fp8_gemm._state["level"] == "hip"
    a, b, sa, sb = operands()
    fake.cutlass_scaled_mm(a, b, sa, sb, BF16)
    fake.cutlass_scaled_mm(a, b, torch.ones(()), torch.ones(()), BF16)
    assert len(hip.calls) == 1 and len(fake.stock.calls) == 1
    assert fp8_gemm.install(fake, level="hip", check=False)                # idempotent: not wrapped twice
    assert fake.cutlass_scaled_mm.__wrapped__ is fake.stock


def test_install_levels(monkeypatch):
    monkeypatch.setattr(fp8_gemm, "_state", dict(fp8_gemm._state))
    with pytest.raises(ValueError):
        fp8_gemm.install(FakeOps(), level="cutlass")
    fake = FakeOps()
    assert not fp8_gemm.install(fake, level="off")
    assert fake.cutlass_scaled_mm is fake.stock
    assert fp8_gemm.install(fake, level="tensor32", check=False)
    assert fp8_gemm._state["level"] == "tensor32" and not fp8_gemm._state["fused"]


def test_route_order_router_then_hook_then_kernel(monkeypatch):
    hip, two = Recorder("hip"), Recorder("two")
    monkeypatch.setattr(fp8_gemm, "scaled_mm_fused", hip)
    monkeypatch.setattr(fp8_gemm, "scaled_mm_tensor32", two)
    a, b, sa, sb = operands()
    order = []
    fp8_gemm.set_router(lambda *args: order.append("router"))
    fp8_gemm.set_stash_hook(lambda *args: order.append("hook"))
    fp8_gemm.route(a, b, sa, sb, BF16)
    assert order == ["router", "hook"] and len(hip.calls) == 1
    fp8_gemm.clear_hooks()
    fp8_gemm.set_router(lambda *args: torch.zeros(1))
    fp8_gemm.set_stash_hook(lambda *args: pytest.fail("hook after a router took the call"))
    assert fp8_gemm.route(a, b, sa, sb, BF16).shape == (1,)
    fp8_gemm.clear_hooks()
    monkeypatch.setitem(fp8_gemm._state, "fused", False)
    fp8_gemm.route(a, b, sa, sb, BF16)
    assert len(two.calls) == 1
    stand_in = Recorder("stand_in")
    fp8_gemm.route(a, b, sa, sb, BF16, two_pass=stand_in)
    assert len(stand_in.calls) == 1 and len(two.calls) == 1


def test_register_once():
    f = lambda *args: None  # noqa: E731
    fp8_gemm.set_router(f)
    fp8_gemm.set_router(f)
    fp8_gemm.set_stash_hook(f)
    fp8_gemm.set_stash_hook(f)
    assert fp8_gemm._routers == [f] and fp8_gemm._stash_hooks == [f]


def test_eligible_call_never_falls_back_to_cpu():
    a, b, sa, sb = operands()
    with pytest.raises(ValueError, match="GPU only"):
        fp8_gemm.scaled_mm_fused(a, b, sa, sb, BF16)
    with pytest.raises(ValueError, match="GPU only"):
        fp8_gemm.scaled_mm_tensor32(a, b, sa, sb, BF16)


def test_vec_scales():
    sa, sb = fp8_gemm._vec_scales(torch.tensor(2.0), torch.arange(4.0).view(1, 4), 3, 4)
    assert sa.tolist() == [2.0, 2.0, 2.0] and sb.tolist() == [0.0, 1.0, 2.0, 3.0]
    assert sa.is_contiguous() and sb.is_contiguous()


# ---- a fake DiT block ---------------------------------------------------------------------------------------------

class FakeQuant:
    """Stands in for vLLM's QuantFP8 (attributes read by the planner; forward is the 'stock' quant)."""
    def __init__(self, static=False):
        self.static = static
        self.use_per_token_if_dynamic = True
        self.is_group_quant = False
        self.num_token_padding = None
        self.calls = 0

    def forward(self, x, scale=None, scale_ub=None):
        self.calls += 1
        return ("stock", x), torch.ones(x.shape[0], 1)

    __call__ = lambda self, *a, **k: type(self).forward(self, *a, **k)  # noqa: E731


class FakeLinear(torch.nn.Module):
    def __init__(self, k, n, ops_module):
        super().__init__()
        self.weight = torch.nn.Parameter(torch.zeros(n, k).to(E4M3).t(), requires_grad=False)   # [K, N], b.t() contig
        self.weight_scale = torch.ones(n)
        self.output_size_per_partition = n
        self.quant_method = type("QM", (), {})()
        self.quant_method.fp8_linear = type("K", (), {})()
        self.quant_method.fp8_linear.quant_fp8 = FakeQuant()
        self.ops = ops_module

    def forward(self, x):
        a = torch.zeros(x.shape[0], self.weight.shape[0]).to(E4M3)
        return self.ops.cutlass_scaled_mm(a, self.weight, torch.ones(x.shape[0], 1), self.weight_scale, BF16), None


class FakeMLP(torch.nn.Module):
    def __init__(self, ops_module, k=64, f=32):
        super().__init__()
        self.fc1 = FakeLinear(k, 2 * f, ops_module)
        self.fc2 = FakeLinear(f, k, ops_module)
        self.act_calls = 0

    def act_fn(self, h):
        self.act_calls += 1
        return h[:, : h.shape[1] // 2]

    def forward(self, x):
        h, _ = self.fc1(x)
        h = self.act_fn(h)
        out, _ = self.fc2(h)
        return out


class FakeAttn(torch.nn.Module):
    def __init__(self, ops_module, k=64):
        super().__init__()
        self.qkv_proj = FakeLinear(k, 3 * k, ops_module)
        self.out_proj = FakeLinear(k, k, ops_module)


class FakeBlock(torch.nn.Module):
    def __init__(self, ops_module):
        super().__init__()
        self.attn = FakeAttn(ops_module)
        self.mlp = FakeMLP(ops_module)
        self.seen = None

    def forward(self, x):
        self.seen = dict(getattr(fp8_hip._tls, "want", None) or {})
        y, _ = self.attn.qkv_proj(x)
        z, _ = self.attn.out_proj(x)
        return self.mlp(x)


# ---- router -------------------------------------------------------------------------------------------------------

def test_router_block_want_and_forward(monkeypatch):
    fake = FakeOps()
    monkeypatch.setattr(fp8_gemm, "_state", dict(fp8_gemm._state))
    fp8_gemm.install(fake, level="hip", check=False)
    hip = Recorder("hip")
    monkeypatch.setattr(fp8_gemm, "scaled_mm_fused", hip)
    routed = Recorder("routed")
    monkeypatch.setattr(fp8_hip, "scaled_mm", routed)
    blk = FakeBlock(fake)
    want = fp8_hip.block_want(blk)
    assert sorted(want.values()) == ["fc1", "out", "qkv"]
    assert (blk.attn.qkv_proj.weight.data_ptr(), tuple(blk.attn.qkv_proj.weight.shape)) in want
    fp8_gemm.set_router(fp8_hip.route)
    fwd = fp8_hip.make_block_forward(FakeBlock.forward)
    fwd(blk, torch.zeros(8, 64))
    assert sorted(blk.seen.values()) == ["fc1", "out", "qkv"]
    assert len(routed.calls) == 3 and len(hip.calls) == 1                  # fc2 is not a router site
    assert getattr(fp8_hip._tls, "want", None) is None                     # restored after the forward
    blk.forward(torch.zeros(8, 64))                                       # outside the wrapper: nothing routed
    assert len(routed.calls) == 3 and len(hip.calls) == 5


def test_router_declines_when_off(monkeypatch):
    monkeypatch.setitem(fp8_hip._state, "ok", False)
    a, b, sa, sb = operands()
    fp8_hip._tls.want = {(b.data_ptr(), tuple(b.shape)): "qkv"}
    try:
        assert fp8_hip.route(a, b, sa, sb, BF16, None) is None
    finally:
        fp8_hip._tls.want = None


def test_router_launch_error_disables(monkeypatch):
    monkeypatch.setitem(fp8_hip._state, "ok", True)

    def boom(*args):
        raise RuntimeError("launch")
    monkeypatch.setattr(fp8_hip, "scaled_mm", boom)
    a, b, sa, sb = operands()
    fp8_hip._tls.want = {(b.data_ptr(), tuple(b.shape)): "out"}
    try:
        assert fp8_hip.route(a, b, sa, sb, BF16, None) is None
        assert not fp8_hip._state["ok"]
    finally:
        fp8_hip._tls.want = None


# ---- SwiGLU stash -------------------------------------------------------------------------------------------------

class FakeFc2Kernel:
    def __init__(self):
        self.calls = []

    def _get_layer_params(self, layer):
        return layer.weight, layer.weight_scale, None, None

    def apply_scaled_mm(self, A, B, out_dtype, As, Bs, bias, output_shape):
        self.calls.append((A, B, As, Bs, output_shape))
        return torch.zeros(output_shape, dtype=out_dtype)


def _swiglu_setup(monkeypatch, level, gemm_ok=True):
    fake = FakeOps()
    monkeypatch.setattr(fp8_gemm, "_state", dict(fp8_gemm._state))
    fp8_gemm.install(fake, level="hip", check=False)
    hip = Recorder("hip")
    monkeypatch.setattr(fp8_gemm, "scaled_mm_fused", hip)
    calls = []
    monkeypatch.setattr(fp8_swiglu, "gemm_swiglu",
                        lambda a, b, sa, sb, bias: calls.append(("gemm_swiglu", a, b, sa, sb)) or
                        torch.zeros(a.shape[0], b.shape[1] // 2, dtype=BF16))
    monkeypatch.setattr(fp8_swiglu, "gemm_swiglu_quant",
                        lambda a, b, sa, sb, bias: calls.append(("gemm_swiglu_quant", a, b, sa, sb)) or
                        (torch.zeros(a.shape[0], b.shape[1] // 2).to(E4M3), torch.ones(a.shape[0], 1)))
    monkeypatch.setattr(fp8_swiglu, "_state", dict(fp8_swiglu._state, gemm_swiglu=gemm_ok))

    class MLP(FakeMLP):
        pass
    assert fp8_swiglu._install_on(MLP, level=level)
    assert not fp8_swiglu._install_on(MLP, level=level)
    fp8_gemm.set_stash_hook(fp8_swiglu._stash_hook)
    return fake, hip, calls, MLP


def test_swiglu_level1_stashes_operands(monkeypatch):
    fake, hip, calls, MLP = _swiglu_setup(monkeypatch, 1)
    mlp = MLP(fake)
    out = mlp(torch.zeros(8, 64))
    assert [c[0] for c in calls] == ["gemm_swiglu"]
    _, a, b, sa, sb = calls[0]
    assert b is mlp.fc1.weight and sa.shape == (8,) and sb.shape == (64,)
    assert mlp.act_calls == 0 and len(hip.calls) == 1 and out.shape == (8, 64)   # fc2 through kernel 2
    assert not getattr(fp8_swiglu._tls, "stash_next", False)


def test_swiglu_level2_feeds_fc2_directly(monkeypatch):
    fake, hip, calls, MLP = _swiglu_setup(monkeypatch, 2)
    kcls = FakeFc2Kernel
    monkeypatch.setitem(fp8_swiglu._state, "fc2_kernel_cls", kcls)
    mlp = MLP(fake)
    mlp.fc2.quant_method.fp8_linear = kern = FakeFc2Kernel()
    out = mlp(torch.zeros(8, 64))
    assert [c[0] for c in calls] == ["gemm_swiglu_quant"] and len(kern.calls) == 1
    assert len(hip.calls) == 0 and out.shape == (8, 64)
    q, B, As, Bs, shape = kern.calls[0]
    assert q.dtype == E4M3 and q.shape == (8, 32) and As.shape == (8, 1) and shape == [8, 64]


def test_swiglu_level2_unsupported_fc2_redoes_fc1(monkeypatch):
    fake, hip, calls, MLP = _swiglu_setup(monkeypatch, 2)
    monkeypatch.setitem(fp8_swiglu._state, "fc2_kernel_cls", FakeFc2Kernel)
    mlp = MLP(fake)                       # fc2's kernel is not a FakeFc2Kernel: no direct call
    mlp(torch.zeros(8, 64))
    assert [c[0] for c in calls] == ["gemm_swiglu_quant"]
    assert mlp.act_calls == 1 and len(hip.calls) == 2   # fc1 redone + fc2


def test_swiglu_hook_declines(monkeypatch):
    fake, hip, calls, MLP = _swiglu_setup(monkeypatch, 1)
    mlp = MLP(fake)
    mlp.fc1.output_size_per_partition = 96   # padded fc1: N != the logical width
    mlp(torch.zeros(8, 64))
    assert calls == [] and mlp.act_calls == 1 and len(hip.calls) == 2
    a, b, sa, sb = operands()
    assert fp8_swiglu._stash_hook(a, b, sa, sb, BF16, None) is None       # not requested


def test_swiglu_without_kernel3_stashes_product(monkeypatch):
    fake, hip, calls, MLP = _swiglu_setup(monkeypatch, 1, gemm_ok=False)
    prods = []
    monkeypatch.setattr(fp8_gemm, "product_fp32", lambda a, b: prods.append(1) or torch.zeros(a.shape[0], b.shape[1]))
    monkeypatch.setattr(fp8_swiglu, "scale_swiglu",
                        lambda x32, sa, sb, bias: calls.append(("scale_swiglu",)) or
                        torch.zeros(x32.shape[0], x32.shape[1] // 2, dtype=BF16))
    MLP(fake)(torch.zeros(8, 64))
    assert prods == [1] and [c[0] for c in calls] == ["scale_swiglu"]


def test_swiglu_thread_local():
    seen = []
    fp8_swiglu._tls.stash_next = True
    t = threading.Thread(target=lambda: seen.append(getattr(fp8_swiglu._tls, "stash_next", False)))
    t.start()
    t.join()
    fp8_swiglu._tls.stash_next = False
    assert seen == [False]


# ---- quant stash ----------------------------------------------------------------------------------------------------

def test_dynamic_per_token_rules():
    q = FakeQuant()
    assert fp8_quant_fuse.dynamic_per_token(q)
    for attr, val in (("static", True), ("use_per_token_if_dynamic", False), ("is_group_quant", True),
                      ("num_token_padding", 16)):
        q2 = FakeQuant()
        setattr(q2, attr, val)
        assert not fp8_quant_fuse.dynamic_per_token(q2), attr


def test_kernel1_takes_cpu_tensors_never():
    x = torch.zeros(4, 64, dtype=BF16)
    assert not fp8_quant_fuse.kernel1_takes(x)


def test_pending_matches():
    qobj = FakeQuant()
    ph = torch.empty(6, 32, dtype=BF16)
    p = fp8_quant_fuse.Pending("fc2", ph, 32, "q", "s", qobj, None, lambda t: t.fill_(1))
    assert p.matches(qobj, ph)
    assert p.matches(qobj, ph.view(-1, 32))
    assert not p.matches(FakeQuant(), ph)                   # another instance
    assert not p.matches(qobj, ph[1:])                      # other pointer
    assert not p.matches(qobj, ph.view(12, 16))             # other width
    assert not p.matches(qobj, ph.float())
    assert not p.matches(qobj, torch.empty(6, 32, dtype=BF16))
    assert p.materialize() is ph and bool((ph == 1).all())


def test_quant_forward_consumes_pending_and_materialises(monkeypatch):
    qobj = FakeQuant()
    orig = FakeQuant.forward
    fwd = fp8_quant_fuse.make_quant_forward(orig)
    ph = torch.empty(6, 32, dtype=BF16)
    ctx = fp8_quant_fuse._Ctx(None, {})
    filled = []
    ctx.pending = fp8_quant_fuse.Pending("fc2", ph, 32, "Q", "S", qobj, None, lambda t: filled.append(1))
    fp8_quant_fuse._tls.ctx = ctx
    try:
        assert fwd(qobj, ph) == ("Q", "S") and ctx.pending is None and qobj.calls == 0
        ctx.pending = fp8_quant_fuse.Pending("fc2", ph, 32, "Q", "S", qobj, None, lambda t: filled.append(1))
        other = torch.zeros(6, 32, dtype=BF16)
        (tag, x), _ = fwd(qobj, other)                     # another tensor: stash materialised, stock quant runs
        assert tag == "stock" and x is other and filled == [1] and ctx.pending is None
        ctx.pending = fp8_quant_fuse.Pending("fc2", ph, 32, "Q", "S", qobj, None, lambda t: filled.append(1))
        (tag, _), _ = fwd(qobj, ph, torch.ones(1))         # a static scale: never the stash
        assert tag == "stock" and filled == [1, 1]
    finally:
        fp8_quant_fuse._tls.ctx = None


def test_quant_forward_kernel1_route(monkeypatch):
    monkeypatch.setitem(fp8_quant_fuse._state, "kernel1", True)
    monkeypatch.setattr(fp8_quant_fuse, "kernel1_takes", lambda x: True)
    monkeypatch.setattr(fp8_quant_fuse, "quant", lambda x: ("k1", x))
    fwd = fp8_quant_fuse.make_quant_forward(FakeQuant.forward)
    x = torch.zeros(4, 64, dtype=BF16)
    assert fwd(FakeQuant(), x)[0] == "k1"
    assert fwd(FakeQuant(static=True), x)[0][0] == "stock"
    assert fwd(FakeQuant(), x, None, torch.ones(1))[0][0] == "stock"      # scale_ub given
    monkeypatch.setitem(fp8_quant_fuse._state, "kernel1", False)
    assert fwd(FakeQuant(), x)[0][0] == "stock"


def test_block_forward_materialises_leftover(monkeypatch):
    monkeypatch.setitem(fp8_quant_fuse._state, "quant_cls", FakeQuant)
    fake = FakeOps()
    blk = FakeBlock(fake)
    filled = []

    def body(self, x):
        ctx = fp8_quant_fuse._tls.ctx
        assert set(ctx.plan) == {"fc2"}
        ctx.pending = fp8_quant_fuse.Pending("fc2", torch.empty(2, 32, dtype=BF16), 32, None, None,
                                             ctx.plan["fc2"][1], ctx.plan["fc2"][0], lambda t: filled.append(1))
        return "out"
    fwd = fp8_quant_fuse.make_block_forward(body, ("fc2",))
    assert fwd(blk, None) == "out" and filled == [1]
    assert fp8_quant_fuse._tls.ctx is None


def test_block_plan_reasons(monkeypatch):
    monkeypatch.setitem(fp8_quant_fuse._state, "quant_cls", FakeQuant)
    blk = FakeBlock(FakeOps())
    plan, _ = fp8_quant_fuse.block_plan(blk, ("qkv", "fc2"))
    assert set(plan) == {"qkv", "fc2"}
    blk.mlp.fc2.quant_method.fp8_linear.quant_fp8 = FakeQuant(static=True)
    plan, reason = fp8_quant_fuse.block_plan(blk, ("fc2",))
    assert plan is None and "fc2" in reason
    blk.mlp.fc2.tp_size = 2
    plan, reason = fp8_quant_fuse.block_plan(blk, ("fc2",))
    assert plan is None and "tp_size" in reason


def test_parse_sites():
    assert fp8_quant_fuse.parse_sites("1") == fp8_quant_fuse.SITES
    assert fp8_quant_fuse.parse_sites("fc2, qkv") == ("qkv", "fc2")
    assert fp8_quant_fuse.parse_sites("off") == ()
    assert fp8_consumers.parse_sites("all") == fp8_consumers.SITES


# ---- consumer stash -----------------------------------------------------------------------------------------------

def test_consumer_stash_protocol(monkeypatch):
    monkeypatch.setitem(fp8_gemm._state, "fused", False)
    monkeypatch.setitem(fp8_gemm._state, "level", "tensor32")
    monkeypatch.setattr(fp8_gemm, "product_fp32", lambda a, b: torch.full((a.shape[0], b.shape[1]), 2.0))
    passes = []
    monkeypatch.setattr(fp8_consumers, "scale_pass_into",
                        lambda x32, sa, sb, bias, y: passes.append(x32.shape) or y.fill_(3))
    fake = FakeOps()
    blk = FakeBlock(fake)
    want, _ = fp8_consumers.block_plan(blk, fp8_consumers.SITES)
    assert sorted(want.values()) == ["fc2", "out", "qkv"]
    ctx = fp8_consumers._Ctx(want)
    fp8_consumers._tls.ctx = ctx
    try:
        a, _, sa, _ = operands(M=8, K=64)
        w = blk.attn.out_proj.weight
        ph = fp8_consumers.stash_hook(a, w, sa, blk.attn.out_proj.weight_scale, BF16, None)
        assert ph.shape == (8, 64) and "out" in ctx.pending
        stock = []
        wrapped = fp8_consumers.make_consumer_wrapper("out", lambda *args: stock.append(args) or "stock")
        assert wrapped("residual") == "stock" and passes == [(8, 64)] and not ctx.pending
        assert bool((ph.float() == 3).all())
        ph = fp8_consumers.stash_hook(a, w, sa, blk.attn.out_proj.weight_scale, BF16, None)
        assert ph is None                                   # each weight is stashed once per block
        ctx.want[(w.data_ptr(), tuple(w.shape))] = "out"
        fp8_consumers.stash_hook(a, w, sa, blk.attn.out_proj.weight_scale, BF16, None)
        fp8_consumers.set_fused("out", lambda st, *args: ("fused", st.x32.shape))
        try:
            assert wrapped("residual") == ("fused", (8, 64)) and not ctx.pending
        finally:
            fp8_consumers.set_fused("out", None)
    finally:
        fp8_consumers._tls.ctx = None


def test_consumer_hook_stands_down_at_fused_level():
    a, b, sa, sb = operands()
    fp8_consumers._tls.ctx = fp8_consumers._Ctx({(b.data_ptr(), tuple(b.shape)): "fc2"})
    try:
        assert fp8_consumers.stash_hook(a, b, sa, sb, BF16, None) is None
    finally:
        fp8_consumers._tls.ctx = None


def test_consumer_install_needs_two_pass_level():
    assert fp8_consumers.install(("qkv",), tr=object()) == []


def test_ops_refuse_cpu():
    x = torch.zeros(4, 64, dtype=BF16)
    with pytest.raises(ValueError):
        ops.quant_rows(x)
    with pytest.raises(ValueError):
        ops.silu_mul_quant(x)
