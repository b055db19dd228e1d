"""The HIP kernels against the committed golden fixtures (tests/golden/*.npz, written by make_golden.py from torch's
CPU routines in the reference mirrors' order): bit for bit, with no oracle in the loop."""
import os

import numpy as np
import pytest
import torch

from _util import assert_quant_equal, bits16
from h3_tp2_amd import ops

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def golden(name):
    return np.load(os.path.join(GOLDEN, name))


def bf16_dev(bits, dev):
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).view(torch.bfloat16).to(dev)


@pytest.mark.parametrize("name", ["quant.npz", "amax_sweep.npz"])
def test_quant_golden(cuda, name):
    gd = golden(name)
    q, s = ops.quant_rows(bf16_dev(gd["x"], cuda))
    assert_quant_equal(q, s, gd["q"], gd["scale"])


def test_epilogue_golden(cuda):
    gd = golden("epilogue.npz")
    acc = torch.from_numpy(gd["acc"]).to(cuda)
    sa, sb = torch.from_numpy(gd["sa"]).to(cuda), torch.from_numpy(gd["sb"]).to(cuda)
    y = ops.scale_bias_cast(acc, sa, sb, None, torch.bfloat16)
    assert np.array_equal(bits16(y), gd["y_bf16"])
    y = ops.scale_bias_cast(acc, sa, sb, None, torch.float16)
    assert np.array_equal(bits16(y), gd["y_fp16"])
    y = ops.scale_bias_cast(acc, sa, sb, bf16_dev(gd["bias"], cuda), torch.bfloat16)
    assert np.array_equal(bits16(y), gd["y_bias_bf16"])


def test_swiglu_golden(cuda):
    gd = golden("swiglu.npz")
    x32 = torch.from_numpy(gd["x32"]).to(cuda)
    h = ops.scale_swiglu(x32, torch.from_numpy(gd["sa"]).to(cuda), torch.from_numpy(gd["sb"]).to(cuda))
    hb, want = bits16(h), gd["h"]
    nan = ((want & 0x7F80) == 0x7F80) & ((want & 0x7F) != 0)
    assert np.array_equal(((hb & 0x7F80) == 0x7F80) & ((hb & 0x7F) != 0), nan)
    assert np.array_equal(hb[~nan], want[~nan])


def test_silu_table_golden(cuda):
    tab = ops.silu_table(cuda).cpu().numpy().view(np.uint16)
    want = golden("swiglu.npz")["silu_torch_exp"]
    nan = ((want & 0x7F80) == 0x7F80) & ((want & 0x7F) != 0)
    assert np.array_equal(((tab & 0x7F80) == 0x7F80) & ((tab & 0x7F) != 0), nan)
    assert np.array_equal(tab[~nan], want[~nan])
