"""Whole-tensor accuracy of every GEMM output of the measured configurations, in the form the target states its
tolerance in: max |y - y_exact| / rms(y_exact), where y_exact = sa[m] sb[n] sum_k a[m, k] w[n, k] is the dequantised
product in float64 (unrounded).  Beside it, the same figure for a perfect bf16 output -- the exact product rounded
once to bf16 -- which no bf16 result can beat, and the rms error over rms.

Configurations (seeded synthetic inputs, as bench.py): the single linear (c1), the QKV projection at 960x576 (c2), the
FFN at 1344x768 5 s (c3: kernel 3 and the down projection), the block chain at 1344x768 15 s (c4: QKV, out, kernel 3,
down, each on the previous stage's quantised output), the grouped launch (c5, every group), and the reference's four
H3 linears at M = 18 880.  For kernel 3 the exact value is silu(g) u with g, u the exact scaled products.

The asserted bound: max error within 2 bf16 ulps of the largest exact output (2^-6 max|y_exact| -- a dropped term, a
wrong scale or a transposed operand is orders of magnitude beyond it), and the rms error within 1 % of the rms.  The
per-element bound, and bit-equality with the oracle on integer operands, are asserted by the other GEMM tests.
Run with -s to print the table.
"""
import math

import pytest
import torch

pytestmark = pytest.mark.gpu


def _rows_chunks(M: int, chunk: int = 8192):
    for r0 in range(0, M, chunk):
        yield r0, min(M, r0 + chunk)


class Acc:
    """Running maxima and sums of one output tensor's comparison with its exact value."""

    def __init__(self):
        self.max_err = self.max_floor = self.max_ref = self.ss_ref = self.ss_err = 0.0
        self.n = 0

    def add(self, y: torch.Tensor, ex: torch.Tensor) -> None:
        yy = y.double()
        d = (yy - ex).abs()
        fl = (ex.float().to(torch.bfloat16).double() - ex).abs()
        self.max_err = max(self.max_err, float(d.max()))
        self.max_floor = max(self.max_floor, float(fl.max()))
        self.max_ref = max(self.max_ref, float(ex.abs().max()))
        self.ss_ref += float((ex * ex).sum())
        self.ss_err += float((d * d).sum())
        self.n += ex.numel()

    def report(self, name: str) -> dict:
        rms = math.sqrt(self.ss_ref / self.n)
        r = {"max_err_rms": self.max_err / rms, "bf16_floor_rms": self.max_floor / rms,
             "rms_err_rms": math.sqrt(self.ss_err / self.n) / rms, "max_ref_rms": self.max_ref / rms}
        print(f"\n[tolerance] {name}: max|err|/rms {r['max_err_rms']:.4f}  bf16 floor {r['bf16_floor_rms']:.4f}  "
              f"rms err/rms {r['rms_err_rms']:.5f}  max|y|/rms {r['max_ref_rms']:.2f}", flush=True)
        assert self.max_err <= 2.0 ** -6 * self.max_ref, (name, r)
        assert r["rms_err_rms"] <= 1e-2, (name, r)
        return r


def linear_stats(name, y, a, w, sa, sb):
    """y [M, N] bf16 against sa sb (a @ w.T) in float64, in row chunks."""
    acc = Acc()
    W = w.float().double()
    sbd = sb.reshape(1, -1).double()
    sad = sa.reshape(-1).double()
    for r0, r1 in _rows_chunks(a.shape[0]):
        ex = torch.mm(a[r0:r1].float().double(), W.t()) * sbd * sad[r0:r1].view(-1, 1)
        acc.add(y[r0:r1], ex)
        del ex
    return acc.report(name)


def swiglu_stats(name, h, a, w, sa, sb):
    """h [M, F] bf16 against silu(g) u, g / u the exact scaled gate / up products (w = [gate | up] rows)."""
    acc = Acc()
    F = h.shape[1]
    Wg, Wu = w[:F].float().double(), w[F:].float().double()
    sbd = sb.reshape(-1).double()
    sad = sa.reshape(-1).double()
    for r0, r1 in _rows_chunks(a.shape[0], 4096):
        A = a[r0:r1].float().double()
        s = sad[r0:r1].view(-1, 1)
        g = torch.mm(A, Wg.t()) * sbd[:F].view(1, -1) * s
        u = torch.mm(A, Wu.t()) * sbd[F:].view(1, -1) * s
        acc.add(h[r0:r1], g * torch.sigmoid(g) * u)
        del g, u
    return acc.report(name)


def _linear(x_bf16, N, seed, device):
    from h3_tp2_amd import ops, synthetic
    K = x_bf16.shape[1]
    a, sa = ops.quant_rows(x_bf16)
    w, sb = ops.quant_rows(synthetic.weight(N, K, seed).to(device))
    return a, w, sa, sb.view(-1)


def test_c1_single_linear(cuda):
    from h3_tp2_amd import ops, synthetic
    c = synthetic.CONFIGS["c1_single_linear"]
    x = synthetic.activations(c["M"], c["K"], seed=0, n_out=c["n_out"]).to(cuda)
    a, w, sa, sb = _linear(x, c["N"], 1, cuda)
    linear_stats("c1 2048x3072x3072", ops.gemm(a, w, sa, sb), a, w, sa, sb)


def test_c2_qkv(cuda):
    from h3_tp2_amd import ops, synthetic
    c = synthetic.CONFIGS["c2_qkv_960x576_5s"]
    x = synthetic.activations(c["M"], c["K"], seed=0, n_out=c["n_out"]).to(cuda)
    a, w, sa, sb = _linear(x, c["N"], 1, cuda)
    linear_stats("c2 QKV 16740x3072->9216", ops.gemm(a, w, sa, sb), a, w, sa, sb)


def test_c3_ffn(cuda):
    from h3_tp2_amd import ops, synthetic
    c = synthetic.CONFIGS["c3_ffn_1344x768_5s"]
    M, K, F = c["M"], c["K"], c["F"]
    x = synthetic.activations(M, K, seed=0, n_out=c["n_out"]).to(cuda)
    a, wgu, sa, sgu = _linear(x, 2 * F, 2, cuda)
    h = ops.gemm_swiglu(a, wgu, sa, sgu)
    swiglu_stats("c3 gate/up + SwiGLU 31248x3072->2x8192", h, a, wgu, sa, sgu)
    qh, sh = ops.quant_rows(h)
    wd, sd = ops.quant_rows(synthetic.weight(K, F, 3).to(cuda))
    linear_stats("c3 down 31248x8192->3072", ops.gemm(qh, wd, sh, sd.view(-1)), qh, wd, sh, sd.view(-1))


def test_c4_chain(cuda):
    """The chain as bench.py runs it: each GEMM against the exact product of its own (quantised) inputs."""
    from h3_tp2_amd import ops, synthetic
    c = synthetic.CONFIGS["c4_chain_1344x768_15s"]
    M, H, F = c["M"], c["K"], 8192
    x = synthetic.activations(M, H, seed=0, n_out=c["n_out"]).to(cuda)
    a, w, sa, sb = _linear(x, 3 * H, 1, cuda)
    linear_stats("c4 QKV 91728x3072->9216", ops.gemm(a, w, sa, sb), a, w, sa, sb)
    del x, a, w
    xo = synthetic.activations(M, H, seed=5, n_out=c["n_out"]).to(cuda)
    a, w, sa, sb = _linear(xo, H, 4, cuda)
    y, q, s = ops.gemm_quant(a, w, sa, sb)
    linear_stats("c4 out 91728x3072->3072", y, a, w, sa, sb)
    del xo, a, w, y
    wgu, sgu = ops.quant_rows(synthetic.weight(2 * F, H, 2).to(cuda))
    h = ops.gemm_swiglu(q, wgu, s, sgu.view(-1))
    swiglu_stats("c4 gate/up + SwiGLU 91728x3072->2x8192", h, q, wgu, s, sgu.view(-1))
    qh, sh = ops.quant_rows(h)
    del h, wgu
    wd, sd = ops.quant_rows(synthetic.weight(H, F, 3).to(cuda))
    linear_stats("c4 down 91728x8192->3072", ops.gemm(qh, wd, sh, sd.view(-1)), qh, wd, sh, sd.view(-1))


def test_c5_grouped(cuda):
    from h3_tp2_amd import ops, synthetic
    probs = []
    for i, (M, K, N, no) in enumerate(synthetic.CONFIGS["c5_grouped"]["groups"]):
        x = synthetic.activations(M, K, seed=10 + i, n_out=no).to(cuda)
        a, sa = ops.quant_rows(x)
        w, sb = ops.quant_rows(synthetic.weight(N, K, seed=20 + i).to(cuda))
        probs.append((a, w, sa, sb.view(-1)))
    outs = ops.grouped_gemm(probs)
    for (a, w, sa, sb), y in zip(probs, outs):
        linear_stats(f"c5 group {a.shape[0]}x{a.shape[1]}->{w.shape[0]}", y, a, w, sa, sb)


@pytest.mark.parametrize("name,N,K", [("qkv", 21504, 5376), ("out", 5376, 7168), ("fc1", 28672, 5376),
                                      ("fc2", 5376, 14336)])
def test_h3_linears_18880(cuda, name, N, K):
    """The reference's H3 linears at its 5 s per-rank row count, log-normal activation rows (its probe inputs)."""
    from h3_tp2_amd import ops, synthetic
    M = 18880
    x = synthetic.activations(M, K, seed=31, kind="lognormal").to(cuda)
    a, w, sa, sb = _linear(x, N, 32, cuda)
    if name == "fc1":
        swiglu_stats(f"H3 fc1 + SwiGLU {M}x{K}->2x{N // 2}", ops.gemm_swiglu(a, w, sa, sb), a, w, sa, sb)
    else:
        linear_stats(f"H3 {name} {M}x{K}->{N}", ops.gemm(a, w, sa, sb), a, w, sa, sb)
