"""A stand-in for the transformer module of the MiniMax H3 DiT as the producer-site hooks see it: module-level
``rms_norm_indexed_scale_shift`` / ``indexed_gate_rms_norm_scale_shift`` (the stock producers, called through the
module so a patch takes effect), a ``MiniMaxH3DiTBlock`` whose forward runs norm1 + AdaLN -> QKV projection and the
gated residual + norm2 + AdaLN -> fc1, and FP8 linears whose quant is a ``QuantFP8``-like instance.  Shaped after the
reference's tests/fake_h3_consumers.py (block :300-360, stand-ins :66-84)."""
from __future__ import annotations

import types

import torch


class FakeQuantFP8:
    """Dynamic per-token QuantFP8 stand-in: ``forward`` is the layer's stock quant (set per test with ``impl``)."""
    impl = None

    def __init__(self):
        self.static = False
        self.use_per_token_if_dynamic = True
        self.is_group_quant = False
        self.num_token_padding = None

    def forward(self, x, scale=None, scale_ub=None):  # noqa: ANN001,ANN201
        return type(self).impl(x)

    def __call__(self, x, scale=None, scale_ub=None):  # noqa: ANN001,ANN201
        return type(self).forward(self, x, scale, scale_ub)


class FakeFP8Linear(torch.nn.Module):
    """Records the (q, scale) its quant returned; ``weight`` is [K, 1] (the hooks read K = weight.shape[0], as of
    vLLM's [K, N] layout)."""

    def __init__(self, k: int, n: int, quant_cls):  # noqa: ANN001
        super().__init__()
        self.weight = torch.nn.Parameter(torch.zeros(k, 1), requires_grad=False)
        self.n = n
        self.quant_method = types.SimpleNamespace(fp8_linear=types.SimpleNamespace(quant_fp8=quant_cls()))
        self.seen: list = []

    def forward(self, x):  # noqa: ANN001,ANN201
        q, s = self.quant_method.fp8_linear.quant_fp8(x.reshape(-1, x.shape[-1]), None, None)
        self.seen.append((q, s))
        return x


def make_tr(stock_rms, stock_gate_rms, quant_cls=FakeQuantFP8, eps: float = 1e-6):  # noqa: ANN001,ANN201
    """A fresh transformer module with the given stock producers."""
    tr = types.ModuleType("fake_minimax_h3_transformer")
    tr.rms_norm_indexed_scale_shift = stock_rms
    tr.indexed_gate_rms_norm_scale_shift = stock_gate_rms

    class MiniMaxH3DiTBlock(torch.nn.Module):
        def __init__(self, H: int, w1: torch.Tensor, w2: torch.Tensor):
            super().__init__()
            self.norm1 = types.SimpleNamespace(weight=w1)
            self.norm2 = types.SimpleNamespace(weight=w2)
            self.attn = torch.nn.Module()
            self.attn.qkv_proj = FakeFP8Linear(H, 3 * H, quant_cls)
            self.attn.out_proj = FakeFP8Linear(H, H, quant_cls)
            self.mlp = torch.nn.Module()
            self.mlp.fc1 = FakeFP8Linear(H, 4 * H, quant_cls)
            self.mlp.fc2 = FakeFP8Linear(2 * H, H, quant_cls)

        def forward(self, x, branch, shift, scale, gate, idx):  # noqa: ANN001,ANN201
            h = tr.rms_norm_indexed_scale_shift(x, self.norm1.weight, shift, scale, idx, eps)
            self.attn.qkv_proj(h)
            res, h2 = tr.indexed_gate_rms_norm_scale_shift(x, gate, branch, self.norm2.weight, shift, scale, idx, eps)
            self.mlp.fc1(h2)
            return res

    tr.MiniMaxH3DiTBlock = MiniMaxH3DiTBlock
    return tr
