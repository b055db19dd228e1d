"""Benchmark of the online-FP8 DiT linear path on one MI355X: prints ONE JSON line.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--only WORKLOAD]

Headline workload (``value``): the QKV projection at the 5 s 960x576 token count -- X bf16 [16740, 3072] quantised
per token to e4m3fn (kernel 1), then the scaled FP8 GEMM against the per-channel-quantised QKV weight [9216, 3072]
with a bf16 output (kernel 2).  A step is one quant + one GEMM over the whole token sequence, inputs resident in HBM;
``value`` = 2 M N K / (step time) in TFLOP/s.  ``roofline`` is the GEMM kernel alone against the FP8 dense MFMA peak
(5.0 PFLOP/s), its average launch time measured with HIP events on the launch stream.  The other measured workloads
(the single linear, the fused FFN and the 15 s block chain at 1344x768, the grouped launch, the quant / SwiGLU-tail
passes and the producers with the quant fused in, against the 8 TB/s HBM peak) are reported under ``workloads``.
``cpu_baseline`` times the CPU oracle of the reference's torch CPU path (per-token quant, fp32 product, scaled
epilogue) on the headline workload's full token count on this host's cores, repeated for about 10 s (median run).
The default 100 untimed warm-up steps let the chip's clock settle: over the first few tens of heavy calls the GEMM's
launch time swings between about 345 and 460 us before it steadies.  Synthetic seeded inputs, random-init weights (no
checkpoints).
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "minimax-h3-2x-dgx-spark-tp2_amd"))

METRIC = "FP8 DiT-linear TFLOP/s (% FP8 MFMA peak) + quant/SwiGLU HBM GB/s"
PEAK_TFLOPS = 5000.0          # MI355X dense FP8 MFMA
PEAK_GBS = 8000.0             # MI355X HBM3E


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=100,
                    help="untimed steps first (the chip's clock settles over the first few tens of heavy calls)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--only", default="", help="comma list of workloads (default: all)")
    ap.add_argument("--cpu-rows", type=int, default=0, help="token rows of the CPU baseline sample (0: all)")
    ap.add_argument("--cpu-seconds", type=float, default=10.0, help="repeat the CPU baseline for at least this long")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="also run a 512 MiB device-to-device copy (the known-size kernel that scales PMC byte counts)")
    return ap.parse_args()


def main() -> None:
    args = parse()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: this build runs the online-FP8 path on one GPU only (the full token sequence resident, no "
              "sharding, no collectives); --gpus must be 1", file=sys.stderr)
        sys.exit(2)
    import torch

    from h3_tp2_amd import ops, synthetic

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    ops.init(0)
    stream = torch.cuda.current_stream(dev)
    only = set(filter(None, args.only.split(",")))

    def ev():
        return torch.cuda.Event(enable_timing=True)

    def time_steps(fn, steps, warmup):
        """Total time of `steps` back-to-back calls (ms), after `warmup` untimed ones; synchronised on both sides."""
        for _ in range(warmup):
            fn()
        torch.cuda.synchronize()
        s, e = ev(), ev()
        s.record(stream)
        for _ in range(steps):
            fn()
        e.record(stream)
        e.synchronize()
        torch.cuda.synchronize()
        return s.elapsed_time(e)

    def quantised_weight(N, K, seed):
        w, sw = ops.quant_rows(synthetic.weight(N, K, seed).to(dev))
        return w, sw.view(-1)

    out = {}

    if args.copy_calibration:
        src = torch.empty(512 << 20, device=dev, dtype=torch.uint8).fill_(1)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst

    # ---- headline: QKV projection, 960x576 5 s (M = 31 x 540) ----
    c2 = synthetic.CONFIGS["c2_qkv_960x576_5s"]
    M, K, N = c2["M"], c2["K"], c2["N"]
    x = synthetic.activations(M, K, seed=0, n_out=c2["n_out"]).to(dev)
    w, sw = quantised_weight(N, K, seed=1)
    q = torch.empty((M, K), device=dev, dtype=ops.E4M3)
    sq = torch.empty((M, 1), device=dev, dtype=torch.float32)
    y = torch.empty((M, N), device=dev, dtype=torch.bfloat16)

    def qkv_step():
        ops.quant_rows(x, q, sq)
        ops.gemm(q, w, sq, sw, torch.bfloat16, out=y)

    steps, warm = args.steps, args.warmup
    t_step = time_steps(qkv_step, steps, warm) / steps
    flops = 2.0 * M * N * K
    t_gemm = time_steps(lambda: ops.gemm(q, w, sq, sw, torch.bfloat16, out=y), steps, warm) / steps
    t_quant = time_steps(lambda: ops.quant_rows(x, q, sq), steps, warm) / steps
    value = flops / (t_step * 1e-3) / 1e12
    gemm_tf = flops / (t_gemm * 1e-3) / 1e12
    quant_bytes = 3.0 * M * K + 4.0 * M
    out["qkv_quant"] = {"ms": round(t_quant, 4), "GB/s": round(quant_bytes / (t_quant * 1e-3) / 1e9, 1),
                        "frac_hbm": round(quant_bytes / (t_quant * 1e-3) / 1e9 / PEAK_GBS, 4)}

    traffic = None
    tpath = os.path.join(ROOT, "profiles", "gemm_qkv_960x576_traffic.txt")
    if os.path.exists(tpath):
        for line in open(tpath):
            if line.startswith("traffic_bytes_per_launch:"):
                traffic = float(line.split(":", 1)[1])

    roofline = {"bound": "mfma", "achieved": round(gemm_tf, 1), "peak": PEAK_TFLOPS, "unit": "TFLOP/s",
                "frac": round(gemm_tf / PEAK_TFLOPS, 4), "traffic": traffic,
                "kernel": "gemm_kernel<bf16> (kernel 2: full-tile rounds + half-tile tail)", "launch_ms": round(t_gemm, 4),
                "flops_per_launch": flops}
    del x

    # ---- the other measured workloads ----
    def want(name):
        return not only or name in only

    if want("vendor"):
        # The same GEMM through the vendor library (torch._scaled_mm -> hipBLASLt) on the same fp8 operands and
        # per-token / per-channel scales, bf16 out: the practical reference point for kernel 2 on this chip.
        try:
            sa2, sb2 = sq.view(M, 1), sw.view(1, N)
            t_v = time_steps(lambda: torch._scaled_mm(q, w.t(), sa2, sb2, out_dtype=torch.bfloat16), steps, warm) / steps
            one = torch.ones((), device=dev)
            t_vt = time_steps(lambda: torch._scaled_mm(q, w.t(), one, one, out_dtype=torch.bfloat16), steps, warm) / steps
            out["vendor_gemm_qkv_960x576"] = {
                "library": "torch._scaled_mm (hipBLASLt)",
                "rowwise_scales_TFLOP/s": round(flops / (t_v * 1e-3) / 1e12, 1),
                "tensorwise_scales_TFLOP/s": round(flops / (t_vt * 1e-3) / 1e12, 1),
                "kernel2_TFLOP/s": round(gemm_tf, 1)}
        except Exception as exc:  # noqa: BLE001
            out["vendor_gemm_qkv_960x576"] = {"error": f"{type(exc).__name__}: {str(exc)[:160]}"}

    if want("c1"):
        c = synthetic.CONFIGS["c1_single_linear"]
        M1, K1, N1 = c["M"], c["K"], c["N"]
        x1 = synthetic.activations(M1, K1, seed=0, n_out=c["n_out"]).to(dev)
        w1, s1 = quantised_weight(N1, K1, seed=1)
        q1 = torch.empty((M1, K1), device=dev, dtype=ops.E4M3)
        sq1 = torch.empty((M1, 1), device=dev, dtype=torch.float32)
        y1 = torch.empty((M1, N1), device=dev, dtype=torch.bfloat16)

        def c1_step():
            ops.quant_rows(x1, q1, sq1)
            ops.gemm(q1, w1, sq1, s1, torch.bfloat16, out=y1)
        t = time_steps(c1_step, steps, warm) / steps
        out["c1_single_linear_2048x3072x3072"] = {"ms": round(t, 4),
                                                 "TFLOP/s": round(2.0 * M1 * N1 * K1 / (t * 1e-3) / 1e12, 1)}
        del x1, w1, q1, y1

    if want("c3"):
        c = synthetic.CONFIGS["c3_ffn_1344x768_5s"]
        M3, K3, F3 = c["M"], c["K"], c["F"]
        x3 = synthetic.activations(M3, K3, seed=0, n_out=c["n_out"]).to(dev)
        wgu, sgu = quantised_weight(2 * F3, K3, seed=2)
        wd, sd = quantised_weight(K3, F3, seed=3)
        q3 = torch.empty((M3, K3), device=dev, dtype=ops.E4M3)
        sq3 = torch.empty((M3, 1), device=dev, dtype=torch.float32)
        hws = torch.empty((M3, F3), device=dev, dtype=torch.bfloat16)
        y3 = torch.empty((M3, K3), device=dev, dtype=torch.bfloat16)

        def c3_step():
            ops.quant_rows(x3, q3, sq3)
            qh, sh = ops.gemm_swiglu_quant(q3, wgu, sq3, sgu, h_ws=hws)
            ops.gemm(qh, wd, sh, sd, torch.bfloat16, out=y3)
        t = time_steps(c3_step, steps, warm) / steps
        f3 = 2.0 * M3 * (2 * F3) * K3 + 2.0 * M3 * K3 * F3
        t_gu = time_steps(lambda: ops.gemm_swiglu(q3, wgu, sq3, sgu), steps, warm) / steps
        amax = torch.empty((M3,), device=dev, dtype=torch.float32)
        ops.gemm_swiglu(q3, wgu, sq3, sgu, row_amax=amax)
        hq = torch.empty((M3, F3), device=dev, dtype=ops.E4M3)
        hs = torch.empty((M3, 1), device=dev, dtype=torch.float32)
        h_in = ops.gemm_swiglu(q3, wgu, sq3, sgu)
        t_tail = time_steps(lambda: ops.quant_rows_amax(h_in, amax, hq, hs), steps, warm) / steps
        tail_bytes = 3.0 * M3 * F3 + 4.0 * M3
        gu_in = torch.empty((M3, 2 * F3), device=dev, dtype=torch.bfloat16).normal_()
        t_sq = time_steps(lambda: ops.silu_mul_quant(gu_in), steps, warm) / steps
        sq_bytes = 5.0 * M3 * F3 + 4.0 * M3
        out["c3_ffn_1344x768_5s"] = {
            "ms": round(t, 4), "TFLOP/s": round(f3 / (t * 1e-3) / 1e12, 1),
            "gate_up_swiglu_TFLOP/s": round(2.0 * M3 * 2 * F3 * K3 / (t_gu * 1e-3) / 1e12, 1),
            "swiglu_requant_tail": {"form": "tail pass of the fused epilogue (3 M F + 4 M bytes)",
                                    "GB/s": round(tail_bytes / (t_tail * 1e-3) / 1e9, 1),
                                    "frac_hbm": round(tail_bytes / (t_tail * 1e-3) / 1e9 / PEAK_GBS, 4)},
            "swiglu_requant_standalone": {"form": "bf16 [M, 2F] -> e4m3 [M, F] (5 M F + 4 M bytes)",
                                          "GB/s": round(sq_bytes / (t_sq * 1e-3) / 1e9, 1),
                                          "frac_hbm": round(sq_bytes / (t_sq * 1e-3) / 1e9 / PEAK_GBS, 4)}}
        del x3, wgu, wd, q3, hws, y3, h_in, gu_in, hq

    if want("c4"):
        c = synthetic.CONFIGS["c4_chain_1344x768_15s"]
        M4, K4 = c["M"], c["K"]
        F4 = 8192
        x4 = synthetic.activations(M4, K4, seed=0, n_out=c["n_out"]).to(dev)
        xo = synthetic.activations(M4, K4, seed=5, n_out=c["n_out"]).to(dev)   # attention output stand-in
        wqkv, sqkv = quantised_weight(3 * K4, K4, seed=1)
        wo, so = quantised_weight(K4, K4, seed=4)
        wgu, sgu = quantised_weight(2 * F4, K4, seed=2)
        wd, sd = quantised_weight(K4, F4, seed=3)
        q4 = torch.empty((M4, K4), device=dev, dtype=ops.E4M3)
        s4 = torch.empty((M4, 1), device=dev, dtype=torch.float32)
        yqkv = torch.empty((M4, 3 * K4), device=dev, dtype=torch.bfloat16)
        hws = torch.empty((M4, F4), device=dev, dtype=torch.bfloat16)

        def c4_step():
            ops.quant_rows(x4, q4, s4)                                       # block input -> fp8
            ops.gemm(q4, wqkv, s4, sqkv, torch.bfloat16, out=yqkv)           # QKV (to attention)
            qo, so_ = ops.quant_rows(xo)                                     # attention output -> fp8
            _, qg, sg = ops.gemm_quant(qo, wo, so_, so)                      # out-proj + fused quant
            qh, sh = ops.gemm_swiglu_quant(qg, wgu, sg, sgu, h_ws=hws)       # gate/up + SwiGLU + requant
            ops.gemm_quant(qh, wd, sh, sd)                                   # down + next block's quant
        t = time_steps(c4_step, max(2, steps // 4), max(1, warm // 2)) / max(2, steps // 4)
        f4 = 2.0 * M4 * (3 * K4 * K4 + K4 * K4 + 2 * F4 * K4 + K4 * F4)
        t_q = time_steps(lambda: ops.quant_rows(x4, q4, s4), steps, warm) / steps
        qb = 3.0 * M4 * K4 + 4.0 * M4
        out["c4_chain_1344x768_15s"] = {"ms": round(t, 3), "TFLOP/s": round(f4 / (t * 1e-3) / 1e12, 1),
                                        "quant_3072": {"GB/s": round(qb / (t_q * 1e-3) / 1e9, 1),
                                                       "frac_hbm": round(qb / (t_q * 1e-3) / 1e9 / PEAK_GBS, 4)},
                                        "note": "out-proj input is a seeded bf16 stand-in for the attention output"}
        del x4, xo, wqkv, wo, wgu, wd, q4, yqkv, hws

    if want("c5"):
        groups = synthetic.CONFIGS["c5_grouped"]["groups"]
        probs, xs = [], []
        for i, (Mg, Kg, Ng, no) in enumerate(groups):
            xg = synthetic.activations(Mg, Kg, seed=10 + i, n_out=no).to(dev)
            wg, sg = quantised_weight(Ng, Kg, seed=20 + i)
            qg, sqg = ops.quant_rows(xg)
            probs.append((qg, wg, sqg, sg))
            xs.append(xg)
        t = time_steps(lambda: ops.grouped_gemm(probs), steps, warm) / steps
        f5 = sum(2.0 * Mg * Ng * Kg for Mg, Kg, Ng, _ in groups)
        out["c5_grouped_one_launch"] = {"ms": round(t, 4), "TFLOP/s": round(f5 / (t * 1e-3) / 1e12, 1),
                                        "note": "all four groups' FLOPs counted, the M=2 adaLN group's included"}
        # the M=2 adaLN group alone: bound by reading its fp8 weight (N x K bytes), reported in GB/s
        Mg, Kg, Ng, _ = groups[0]
        qa, wa, sqa, swa = probs[0]
        t2 = time_steps(lambda: ops.gemm(qa, wa, sqa, swa, torch.bfloat16), steps, warm) / steps
        wbytes = float(Ng * Kg)
        out["c5_grouped_one_launch"]["adaLN_M2_alone"] = {
            "ms": round(t2, 4), "GB/s": round(wbytes / (t2 * 1e-3) / 1e9, 1),
            "frac_hbm": round(wbytes / (t2 * 1e-3) / 1e9 / PEAK_GBS, 4),
            "form": f"kernel 2 on [{Mg},{Kg}] x [{Ng},{Kg}]: {Ng // 256} column tiles of 256 x 256 run as half tiles"}
        del probs, xs

    if want("producers"):
        # The quant fused into its producers: norm1 + AdaLN -> QKV input at the 960x576 5 s token count, the gated
        # residual + norm2 + AdaLN -> fc1 input at the 1344x768 5 s count; H = 3072, a [6, 6H] modulation table.
        H = K
        gen = torch.Generator(device=dev).manual_seed(7)
        res = {}
        for name, Mp, gate in (("qkv_rms_quant_16740x3072", M, False), ("fc1_gate_rms_quant_31248x3072",
                                                                         synthetic.CONFIGS["c3_ffn_1344x768_5s"]["M"],
                                                                         True)):
            xp = (torch.randn(Mp, H, device=dev, generator=gen)
                  * torch.exp(torch.randn(Mp, 1, device=dev, generator=gen))).to(torch.bfloat16)
            wn = (1.0 + 0.1 * torch.randn(H, device=dev, generator=gen)).to(torch.bfloat16)
            ada = torch.randn(6, 6 * H, device=dev, generator=gen).to(torch.bfloat16)
            shp, scp, gtp = ada[:, :H], ada[:, H:2 * H], ada[:, 2 * H:3 * H]
            idx = torch.randint(0, 6, (Mp,), device=dev, generator=gen)
            if gate:
                br = torch.randn(Mp, H, device=dev, generator=gen).to(torch.bfloat16)
                fused = lambda: ops.gate_rms_quant(xp, gtp, br, wn, shp, scp, idx, 1e-6)  # noqa: E731

                def unfused():
                    _, hh = ops.indexed_gate_rms_norm_scale_shift(xp, gtp, br, wn, shp, scp, idx, 1e-6)
                    ops.quant_rows(hh)
                nbytes = 7.0 * Mp * H + 4.0 * Mp          # residual, branch, residual_out (bf16) + q + scale
            else:
                fused = lambda: ops.rms_quant(xp, wn, shp, scp, idx, 1e-6)  # noqa: E731

                def unfused():
                    ops.quant_rows(ops.rms_norm_indexed_scale_shift(xp, wn, shp, scp, idx, 1e-6))
                nbytes = 3.0 * Mp * H + 4.0 * Mp          # x (bf16) + q + scale
            t_f = time_steps(fused, steps, warm) / steps
            t_u = time_steps(unfused, steps, warm) / steps
            res[name] = {"ms": round(t_f, 4), "GB/s": round(nbytes / (t_f * 1e-3) / 1e9, 1),
                         "frac_hbm": round(nbytes / (t_f * 1e-3) / 1e9 / PEAK_GBS, 4),
                         "unfused_ms": round(t_u, 4), "speedup_vs_unfused": round(t_u / t_f, 3)}
            del xp, ada, idx
            if gate:
                del br
        out["producers_fused_quant"] = res

    if want("consumers"):
        # The consumers of the two-pass GEMM's fp32 product with the scale pass fused in: qk-RMSNorm + RoPE of the
        # QKV output (960x576 5 s, 24 q + 24 k heads of 128, plus the v columns' scale pass), the gated residual +
        # RMS/AdaLN of the out projection and indexed_gate of fc2 (1344x768 5 s, H = 3072).
        from h3_tp2_amd import fp8_consumers as fc
        gen = torch.Generator(device=dev).manual_seed(9)
        res = {}
        T, Hq = M, K // 128
        x32 = torch.randn(T, N, device=dev, generator=gen) * 3000
        sa_t = torch.rand(T, device=dev, generator=gen) * 1e-3 + 1e-4
        sb_t = torch.rand(N, device=dev, generator=gen) * 1e-3 + 1e-4
        wq = (1 + 0.1 * torch.randn(128, device=dev, generator=gen)).to(torch.bfloat16)
        pos = torch.rand(T, 1, device=dev, generator=gen) * 500 * torch.exp(-torch.arange(48, device=dev) / 8.0)
        rope = torch.cat((torch.cos(pos), torch.sin(pos)), dim=-1)
        st = fc.Stash(x32, sa_t, sb_t, None, torch.empty((T, N), device=dev, dtype=torch.bfloat16))
        t_qk = time_steps(lambda: fc.qk_norm_rope_fused(st, Hq, Hq, 128, wq, wq, rope, 1e-6), steps, warm) / steps
        qk_bytes = T * N * 4.0 + T * N * 2.0                         # product in, q / k / v bf16 out
        res["qkv_qk_norm_rope_16740x9216"] = {"ms": round(t_qk, 4), "GB/s": round(qk_bytes / (t_qk * 1e-3) / 1e9, 1),
                                              "frac_hbm": round(qk_bytes / (t_qk * 1e-3) / 1e9 / PEAK_GBS, 4)}
        del x32, st
        Mc, H = synthetic.CONFIGS["c3_ffn_1344x768_5s"]["M"], K
        x32 = torch.randn(Mc, H, device=dev, generator=gen) * 3000
        sa_c = torch.rand(Mc, device=dev, generator=gen) * 1e-3 + 1e-4
        sb_c = torch.rand(H, device=dev, generator=gen) * 1e-3 + 1e-4
        resid = torch.randn(Mc, H, device=dev, generator=gen).to(torch.bfloat16)
        wn = (1.0 + 0.1 * torch.randn(H, device=dev, generator=gen)).to(torch.bfloat16)
        ada = torch.randn(6, 6 * H, device=dev, generator=gen).to(torch.bfloat16)
        idx = torch.randint(0, 6, (Mc,), device=dev, generator=gen)
        st = fc.Stash(x32, sa_c, sb_c, None, torch.empty((Mc, H), device=dev, dtype=torch.bfloat16))
        t_out = time_steps(lambda: fc.gate_rms_fused(st, resid, ada[:, 2 * H:3 * H], wn, ada[:, :H], ada[:, H:2 * H],
                                                     idx, 1e-6), steps, warm) / steps
        out_bytes = Mc * H * (4.0 + 2 + 2 + 2)                       # product, residual in; residual_out, h out
        t_fc2 = time_steps(lambda: fc.gate_fused(st, resid, ada[:, 5 * H:], idx), steps, warm) / steps
        fc2_bytes = Mc * H * (4.0 + 2 + 2)                           # product, x in; out
        res["out_gate_rms_31248x3072"] = {"ms": round(t_out, 4), "GB/s": round(out_bytes / (t_out * 1e-3) / 1e9, 1),
                                          "frac_hbm": round(out_bytes / (t_out * 1e-3) / 1e9 / PEAK_GBS, 4)}
        res["fc2_indexed_gate_31248x3072"] = {"ms": round(t_fc2, 4),
                                              "GB/s": round(fc2_bytes / (t_fc2 * 1e-3) / 1e9, 1),
                                              "frac_hbm": round(fc2_bytes / (t_fc2 * 1e-3) / 1e9 / PEAK_GBS, 4)}
        del x32, st, resid, ada
        out["consumers_of_fp32_product"] = res

    # ---- CPU baseline: the oracle of the reference's torch CPU path on the headline workload ----
    cpu = None
    if not args.no_cpu:
        sys.path.insert(0, ROOT)
        import numpy as np

        from oracle import oracle as O
        rows = min(args.cpu_rows, M) if args.cpu_rows > 0 else M
        xs = synthetic.activations(M, K, seed=0, n_out=c2["n_out"])[:rows]
        xb = xs.view(torch.int16).numpy().view(np.uint16)
        wb = synthetic.weight(N, K, seed=1).view(torch.int16).numpy().view(np.uint16)
        wq, swq = O.quant_rows(wb)
        O.linear(xb[:16], wq, swq)                                           # warm-up
        runs = []
        while len(runs) < 3 or sum(runs) < args.cpu_seconds:
            t0 = time.perf_counter()
            O.linear(xb, wq, swq)
            runs.append(time.perf_counter() - t0)
        med = sorted(runs)[len(runs) // 2]
        t_full = med * M / rows
        threads = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
        cpu = {"value": round(flops / t_full / 1e12, 5), "unit": "TFLOP/s", "cores": threads, "kind": "port",
               "sample": f"oracle per-token quant + numpy fp32 product + C epilogue on {rows} of {M} token rows, "
                         f"median of {len(runs)} runs ({med:.2f} s each, {sum(runs):.1f} s in all)"
                         + ("" if rows == M else f", scaled linearly to {M} rows"),
               "host_cpu_count": os.cpu_count()}

    line = {"metric": METRIC, "value": round(value, 1), "unit": "TFLOP/s", "n_gpus": 1, "steps": steps,
            "warmup": warm, "ms_per_step": round(t_step, 4), "higher_is_better": True, "scaling": "weak",
            "vs_baseline": None, "dtype": "e4m3", "data": "synthetic (seeded N(0,1) activations with x40 outlier "
            "channels, random-init N(0,0.02) weights)",
            "config": {"workload": "qkv_960x576_5s: quant X[16740,3072] + FP8 GEMM vs W[9216,3072], bf16 out",
                       "M": M, "K": K, "N": N, "parallelism": "single GPU"},
            "roofline": roofline, "cpu_baseline": cpu, "workloads": out}
    print(json.dumps(line))


if __name__ == "__main__":
    main()
