"""The host protocols on the GPU, through the real kernels: the MLP stash protocol (fp8_swiglu levels 1 and 2) and the
block router (fp8_hip), on stand-in layers that hold real FP8 weights and call the dispatcher the way vLLM's FP8
linear does (per-token quant of the input, then ``cutlass_scaled_mm``).  Every tensor that crosses the protocol -- the
fused SwiGLU row h, fc2's quantised input and scale, the routed GEMM outputs -- is compared with the oracle applied to
the kernel's own fp32 accumulator (read back through the raw-accumulator mode), bit for bit.  Pattern of the
reference's tests/test_fp8_swiglu.py:131 (the MLP forward paths on the GPU) and tests/test_fp8_cutlass_gpu.py:77-85
(the router on a side stream)."""
import threading

import numpy as np
import pytest
import torch

from _util import assert_quant_equal, bits16, f32, oracle_quant
from h3_tp2_amd import fp8_gemm, fp8_hip, fp8_swiglu, ops, synthetic
from oracle import oracle as O

pytestmark = pytest.mark.gpu
BF16 = torch.bfloat16
E4M3 = torch.float8_e4m3fn


class DispatchOps:
    """Stands in for vLLM's ``_custom_ops``: the stock op must never run for an eligible call."""

    def __init__(self):
        self.stock = 0

    def cutlass_scaled_mm(self, a, b, scale_a, scale_b, out_dtype, bias=None):
        self.stock += 1
        raise AssertionError("stock cutlass_scaled_mm reached")


class Fp8Linear(torch.nn.Module):
    """An FP8 linear as vLLM runs it: kernel 1 quantises the input per token, then ``ops.cutlass_scaled_mm`` with the
    per-channel weight scale.  ``weight`` is vLLM's [K, N] view of the [N, K] e4m3 weight; ``seen`` records the
    (q, scale) each call quantised."""

    def __init__(self, n: int, k: int, seed: int, ops_module, device):
        super().__init__()
        w, sw = ops.quant_rows(synthetic.weight(n, k, seed).to(device))
        self.register_buffer("w_nk", w)
        self.weight = w.t()
        self.weight_scale = sw.view(-1)
        self.output_size_per_partition = n
        self.ops = ops_module
        self.seen = []
        self.quant_method = type("QM", (), {})()
        self.quant_method.fp8_linear = None

    def forward(self, x):
        q, s = ops.quant_rows(x.reshape(-1, x.shape[-1]).contiguous())
        self.seen.append((q, s))
        y = self.ops.cutlass_scaled_mm(q, self.weight, s, self.weight_scale, BF16)
        return y.view(*x.shape[:-1], y.shape[-1]), None


class Fc2Kernel:
    """fc2's scaled-mm kernel: records the pre-quantised input it is handed (level 2) and runs kernel 2 on it."""

    def __init__(self):
        self.calls = []

    def _get_layer_params(self, layer):
        return layer.weight, layer.weight_scale, None, None

    def apply_scaled_mm(self, A, B, out_dtype, As, Bs, bias, output_shape):
        self.calls.append((A, As))
        return ops.scaled_mm(A, B, As, Bs, out_dtype).view(output_shape)


class MLP(torch.nn.Module):
    def __init__(self, ops_module, device, hidden=3072, ffn=2048):
        super().__init__()
        self.fc1 = Fp8Linear(2 * ffn, hidden, 31, ops_module, device)
        self.fc2 = Fp8Linear(hidden, ffn, 32, ops_module, device)
        self.fc2.quant_method.fp8_linear = Fc2Kernel()
        self.act_calls = 0

    def act_fn(self, h):
        self.act_calls += 1
        raise AssertionError("the stock activation ran although fc1 was stashed")

    def forward(self, x):
        h, _ = self.fc1(x)
        h = self.act_fn(h)
        out, _ = self.fc2(h)
        return out


@pytest.fixture
def dispatch(cuda, monkeypatch):
    monkeypatch.setattr(fp8_gemm, "_state", dict(fp8_gemm._state))
    fake = DispatchOps()
    assert fp8_gemm.install(fake, level="hip", check=True)
    yield fake
    fp8_gemm.clear_hooks()


def _kernel_acc(q, s, lin):
    """The kernel's own fp32 accumulator of ``lin``'s GEMM on (q, s) (the raw-accumulator mode)."""
    return f32(ops.gemm(q, lin.w_nk, s, lin.weight_scale, torch.float32))


@pytest.mark.parametrize("level", [1, 2])
def test_mlp_stash_protocol_on_the_kernels(cuda, dispatch, monkeypatch, level):
    monkeypatch.setattr(fp8_swiglu, "_state", dict(fp8_swiglu._state, fc2_kernel_cls=Fc2Kernel))
    monkeypatch.setattr(fp8_swiglu, "_tls", threading.local())
    monkeypatch.setattr(fp8_swiglu, "_stats", dict.fromkeys(fp8_swiglu._stats, 0))
    assert fp8_swiglu.probe_gemm_swiglu(cuda)

    class WrappedMLP(MLP):
        pass
    assert fp8_swiglu._install_on(WrappedMLP, level=level)
    fp8_gemm.set_stash_hook(fp8_swiglu._stash_hook)
    mlp = WrappedMLP(dispatch, cuda)
    M = 1200
    x = synthetic.activations(M, 3072, seed=8, n_out=3).to(cuda)
    out = mlp(x)
    torch.cuda.synchronize()
    assert dispatch.stock == 0 and mlp.act_calls == 0
    (qx, sx), = mlp.fc1.seen                                    # fc1's input: kernel 1 = the oracle's quant
    assert_quant_equal(qx, sx, *oracle_quant(x.cpu()))
    acc1 = _kernel_acc(qx, sx, mlp.fc1)
    sw1 = f32(mlp.fc1.weight_scale)
    if level == 2:
        assert fp8_swiglu.stats()["fused_quant"] == 1 and fp8_swiglu.stats()["fc2_direct"] == 1
        (q2, s2), = mlp.fc2.quant_method.fp8_linear.calls        # fc2's input handed over pre-quantised
        assert mlp.fc2.seen == []                                # ... and fc2's own quant never ran
        q_ref, s_ref = O.scale_swiglu_quant(acc1, f32(sx), sw1)
        assert_quant_equal(q2, s2, q_ref, s_ref)
    else:
        assert fp8_swiglu.stats()["fused"] == 1
        (q2, s2), = mlp.fc2.seen                                # fc2 quantised the fused h itself
        h_ref = O.scale_swiglu(acc1, f32(sx), sw1)
        assert_quant_equal(q2, s2, *O.quant_rows(h_ref))
    acc2 = _kernel_acc(q2, s2, mlp.fc2)
    y_ref = O.epilogue(acc2, f32(s2), f32(mlp.fc2.weight_scale))
    assert np.array_equal(bits16(out), y_ref)


class Attn(torch.nn.Module):
    def __init__(self, ops_module, device, hidden=3072):
        super().__init__()
        self.qkv_proj = Fp8Linear(3 * hidden, hidden, 41, ops_module, device)
        self.out_proj = Fp8Linear(hidden, hidden, 42, ops_module, device)


class Block(torch.nn.Module):
    """A DiT block's linears in the order of the forward: QKV on x, out on an attention stand-in, fc1 on the out
    projection's output; fc2 is not a router site."""

    def __init__(self, ops_module, device):
        super().__init__()
        self.attn = Attn(ops_module, device)
        self.mlp = torch.nn.Module()
        self.mlp.fc1 = Fp8Linear(2 * 2048, 3072, 43, ops_module, device)
        self.mlp.fc2 = Fp8Linear(3072, 2048, 44, ops_module, device)

    def forward(self, x, attn_out):
        qkv, _ = self.attn.qkv_proj(x)
        o, _ = self.attn.out_proj(attn_out)
        h, _ = self.mlp.fc1(o)
        y, _ = self.mlp.fc2(h[:, :2048].contiguous())
        return qkv, o, h, y


def test_block_router_on_the_kernels(cuda, monkeypatch):
    """fp8_hip routes the block's qkv / out / fc1 GEMMs to kernel 2 (ahead of the dispatcher's two-pass level) while the
    block's forward runs, on a side stream; fc2 and any GEMM outside a block forward go through the two-pass level.
    Both forms give the oracle's epilogue of the kernel's accumulator."""
    monkeypatch.setattr(fp8_gemm, "_state", dict(fp8_gemm._state))
    monkeypatch.setattr(fp8_hip, "_state", dict(fp8_hip._state))
    monkeypatch.setattr(fp8_hip, "_stats", dict.fromkeys(fp8_hip._stats, 0))
    fake = DispatchOps()
    try:
        assert fp8_gemm.install(fake, level="tensor32", check=True)
        two_pass_before = fp8_gemm.stats()["two_pass"]

        class WrappedBlock(Block):
            pass
        tr = type("tr", (), {"MiniMaxH3DiTBlock": WrappedBlock})
        assert fp8_hip.install_sites(tr, check=True)
        blk = WrappedBlock(fake, cuda)
        M = 1000
        x = synthetic.activations(M, 3072, seed=9, n_out=3).to(cuda)
        att = synthetic.activations(M, 3072, seed=10, n_out=3).to(cuda)
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            qkv, o, h, y = blk(x, att)
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        assert fp8_hip.stats()["hip"] == 3 and fake.stock == 0
        assert fp8_gemm.stats()["two_pass"] - two_pass_before == 1            # fc2 only
        assert getattr(fp8_hip._tls, "want", None) is None
        for lin, out in ((blk.attn.qkv_proj, qkv), (blk.attn.out_proj, o), (blk.mlp.fc1, h), (blk.mlp.fc2, y)):
            (q, s), = lin.seen
            ref = O.epilogue(_kernel_acc(q, s, lin), f32(s), f32(lin.weight_scale))
            assert np.array_equal(bits16(out), ref), lin
        qkv_outside, _ = blk.attn.qkv_proj(x)                                 # outside a block forward: two-pass
        torch.cuda.synchronize()
        assert fp8_hip.stats()["hip"] == 3 and torch.equal(qkv_outside.view(torch.int16), qkv.view(torch.int16))
    finally:
        fp8_gemm.clear_hooks()
