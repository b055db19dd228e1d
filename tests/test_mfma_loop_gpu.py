"""The register-only MFMA loop that bench.py uses as the chip's sustained FP8 MFMA rate: it runs through the C ABI,
its sums are finite and depend only on the seed (the same seed twice gives the same bits, another seed other bits),
and the ABI rejects a grid outside its limits."""
import pytest
import torch

from h3_tp2_amd import _lib, ops

pytestmark = pytest.mark.gpu


def test_mfma_loop_runs_and_is_deterministic(cuda):
    out1 = torch.empty(8 * 256, device=cuda)
    out2 = torch.empty_like(out1)
    out3 = torch.empty_like(out1)
    ops.mfma_loop(out1, 50, seed=7)
    ops.mfma_loop(out2, 50, seed=7)
    ops.mfma_loop(out3, 50, seed=8)
    torch.cuda.synchronize()
    assert bool(torch.isfinite(out1).all())
    assert torch.equal(out1.view(torch.int32), out2.view(torch.int32))
    assert not torch.equal(out1.view(torch.int32), out3.view(torch.int32))


def test_mfma_loop_rejects_bad_grid(cuda):
    out = torch.empty(256, device=cuda)
    for blocks, iters in ((0, 1), (70000, 1), (1, 0)):
        with pytest.raises(_lib.H3Fp8Error):
            _lib.call("h3fp8_mfma_loop", out.data_ptr(), blocks, iters, 1, 0)
