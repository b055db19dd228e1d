"""h3fp8_gemm_quant_noalloc -- the GEMM + fused next-layer quant with the row maxima in the library's own static
buffer (no allocation) -- against h3fp8_gemm_quant with a caller workspace, through the C ABI.

Two calls in a row, the second with fewer rows (the buffer keeps the first call's maxima; each call must clear what it
uses), then a call at the buffer's row limit, and the refusals of a call one row past it and of bad shapes."""
import ctypes

import numpy as np
import pytest
import torch

from _util import serving_like

pytestmark = pytest.mark.gpu
E4M3 = torch.float8_e4m3fn


def _call(name, a, w, sa, sb, y, q, s, ws=None):
    from h3_tp2_amd import _lib
    M, K = a.shape
    N = w.shape[0]
    args = [a.data_ptr(), K, w.data_ptr(), K, sa.data_ptr(), 1, sb.data_ptr(), 1, None, y.data_ptr(), N, M, N, K]
    if ws is not None:
        args.append(ws.data_ptr())
    args += [q.data_ptr(), N, s.data_ptr(), torch.cuda.current_stream().cuda_stream]
    _lib.call(name, *args)


def _outputs(M, N, dev):
    return (torch.empty((M, N), device=dev, dtype=torch.bfloat16), torch.empty((M, N), device=dev, dtype=E4M3),
            torch.empty((M,), device=dev))


def _same(a, b):
    return torch.equal(a.contiguous().view(torch.uint8), b.contiguous().view(torch.uint8))


@pytest.mark.parametrize("sizes", [[(3000, 3072, 1024), (700, 3072, 1024)], [(16740, 9216, 3072), (256, 512, 256)]])
def test_noalloc_equals_workspace_form(cuda, sizes):
    for i, (M, N, K) in enumerate(sizes):
        a, w, sa, sb = serving_like(M, N, K, seed=50 + i, device=cuda)
        y0, q0, s0 = _outputs(M, N, cuda)
        ws = torch.full((M,), 3.0, device=cuda)
        _call("h3fp8_gemm_quant", a, w, sa, sb, y0, q0, s0, ws)
        y1, q1, s1 = _outputs(M, N, cuda)
        _call("h3fp8_gemm_quant_noalloc", a, w, sa, sb, y1, q1, s1)
        torch.cuda.synchronize()
        assert _same(y1, y0) and _same(q1, q0) and _same(s1, s0), (M, N, K)


def test_noalloc_at_the_row_limit_and_refusals(cuda):
    from h3_tp2_amd import H3Fp8Error, _lib
    M, N, K = _lib.NOALLOC_MAX_ROWS, 256, 128
    g = torch.Generator(device=cuda).manual_seed(5)
    a = torch.randint(-4, 5, (M, K), generator=g, device=cuda).float().to(E4M3)
    w = torch.randint(-2, 3, (N, K), generator=g, device=cuda).float().to(E4M3)
    sa = torch.rand(M, generator=g, device=cuda) * 1e-2 + 1e-3
    sb = torch.rand(N, generator=g, device=cuda) * 1e-2 + 1e-3
    y0, q0, s0 = _outputs(M, N, cuda)
    _call("h3fp8_gemm_quant", a, w, sa, sb, y0, q0, s0, torch.empty(M, device=cuda))
    y1, q1, s1 = _outputs(M, N, cuda)
    _call("h3fp8_gemm_quant_noalloc", a, w, sa, sb, y1, q1, s1)
    torch.cuda.synchronize()
    assert _same(y1, y0) and _same(q1, q0) and _same(s1, s0)
    # one row past the limit is refused before any launch, with the outputs untouched
    a2 = torch.zeros((M + 1, K), device=cuda, dtype=E4M3)
    y2, q2, s2 = _outputs(M + 1, N, cuda)
    s2.fill_(-1.0)
    with pytest.raises(H3Fp8Error, match="exceeds"):
        _call("h3fp8_gemm_quant_noalloc", a2, w, torch.ones(M + 1, device=cuda), sb, y2, q2, s2)
    torch.cuda.synchronize()
    assert bool((s2 == -1.0).all())
    L = _lib.load()
    assert L.h3fp8_gemm_quant_noalloc(None, 32, None, 32, None, 1, None, 1, None, None, 32, 4, 32, 32, None, 32,
                                      None, None) == -22
    assert b"null output" in L.h3fp8_last_error()
    dummy = ctypes.c_void_p(256)                  # never dereferenced: the shape check refuses first
    assert L.h3fp8_gemm_quant_noalloc(None, 32, None, 32, None, 1, None, 1, None, None, 32, 4, 24, 24, dummy, 32,
                                      dummy, None) == -22
    assert b"multiples of 16" in L.h3fp8_last_error()


def test_noalloc_captured_in_a_graph_replays_bitwise(cuda):
    """The entry point captured in a HIP graph (torch.cuda.graph): the row maxima are cleared by a fill kernel, so no
    memset node is recorded.  Three replays, each after the outputs were overwritten eagerly and other eager GEMM work
    ran, with a synchronisation in between; every replay equals the workspace form bit for bit."""
    from h3_tp2_amd import ops
    M, N, K = 3000, 3072, 1024
    a, w, sa, sb = serving_like(M, N, K, seed=77, device=cuda)
    y0, q0, s0 = _outputs(M, N, cuda)
    _call("h3fp8_gemm_quant", a, w, sa, sb, y0, q0, s0, torch.empty(M, device=cuda))
    y1, q1, s1 = _outputs(M, N, cuda)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        _call("h3fp8_gemm_quant_noalloc", a, w, sa, sb, y1, q1, s1)
    a2, w2, sa2, sb2 = serving_like(700, 1024, 512, seed=78, device=cuda)
    for rep in range(3):
        y1.fill_(float("nan"))
        q1.view(torch.uint8).fill_(0x7F)
        s1.fill_(-1.0)
        ops.gemm_quant(a2, w2, sa2, sb2)                    # other eager work between the replays
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert _same(y1, y0) and _same(q1, q0) and _same(s1, s0), f"replay {rep}"
    del g
