"""Benchmark of the online-FP8 DiT linear path on one MI355X: prints ONE JSON line.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--preroll-s S] [--no-cpu] [--only WORKLOADS]

Headline workload (``value``): the full DiT block linear chain at the 15 s 1344x768 token count (M = 91 728 tokens,
hidden 3072), the set the target is quoted on.  One step is: X -> per-token quant (kernel 1) -> QKV GEMM [3072 -> 9216]
(kernel 2); the attention-output stand-in -> quant -> out-projection [3072 -> 3072] whose epilogue reduces the row
maxima, and the quant tail from them; gate/up GEMM [3072 -> 2 x 8192] with the SwiGLU epilogue (kernel 3) and its
requant tail; down GEMM [8192 -> 3072] with the next block's quant fused the same way.  ``value`` = the chain's 2 M (3
H^2 + H^2 + 2 F H + F H) FLOPs / step time, in TFLOP/s, inputs resident in HBM.  The timed steps run with no event
inside; the same number of steps again with HIP events between every two launches on the launch stream gives the
per-kernel averages (``breakdown``) and ``roofline``: ``roofline`` is kernel 3 (gate/up + SwiGLU, 44 % of the chain's
FLOPs) against the 5.0 PFLOP/s FP8 dense MFMA peak.  Before the warm-up steps an explicit pre-roll runs the chain for
``--preroll-s`` seconds: the chip's clock moves over the first heavy calls, and the pre-roll makes the timed steps
independent of how short the warm-up is.  The other measured workloads (the QKV projection at 960x576, the single
linear, the FFN at 1344x768 5 s, the grouped launch, the reference's four H3 linears at its per-rank M = 42 848, the
out projection's input quantised from a Ulysses receive buffer, the host cost of one dispatched call, the producers /
consumers passes and the fc1 stash forms of the two-pass MLP (fp32 gate/up product -> SwiGLU, and -> SwiGLU + requant),
the vendor GEMM, the socket power and clock of each chain launch beside a register-only MFMA loop) are reported under
``workloads``.  ``cpu_baseline`` times the reference's torch CPU path (oracle/torch_path.py) of the same chain on a row
sample, on this host's cores.  Synthetic seeded inputs, random-init weights (no checkpoints).
"""
from __future__ import annotations

import argparse
import json
import os
import subprocess
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
    ap.add_argument("--steps", type=int, default=30)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--preroll-s", type=float, default=1.0,
                    help="seconds of untimed chain steps before the warm-up (lets the chip's clock settle)")
    ap.add_argument("--settle-s", type=float, default=0.25,
                    help="seconds of untimed calls before each other workload's warm-up (its inputs are made on the "
                         "host while the GPU idles, so the clock drops between workloads)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--only", default="", help="comma list of the extra workloads to run (default: all; 'none': none)")
    ap.add_argument("--cpu-rows", type=int, default=2048, help="token rows of the CPU baseline sample")
    ap.add_argument("--cpu-seconds", type=float, default=10.0, help="repeat the CPU baseline for at least this long")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="also run a 512 MiB device-to-device copy (the known-size kernel that scales PMC byte counts)")
    ap.add_argument("--power-s", type=float, default=2.0,
                    help="seconds each launch of the power / clock workload runs back to back")
    return ap.parse_args()


def smi_sample(smi: str) -> tuple[float, float]:
    """(socket power W, mean gfx clock MHz over the XCDs) of GPU 0 from one `amd-smi metric -p -c --json` call."""
    r = subprocess.run([smi, "metric", "-p", "-c", "--json"], capture_output=True, text=True, timeout=10)
    o = json.loads(r.stdout)
    g = o["gpu_data"][0] if isinstance(o, dict) else o[0]
    clks = [float(v["clk"]["value"]) for k, v in g["clock"].items()
            if k.startswith("gfx_") and isinstance(v, dict) and isinstance(v.get("clk"), dict)]
    return float(g["power"]["socket_power"]["value"]), sum(clks) / len(clks)


def host_cpu() -> dict:
    """CPU model, physical cores and the threads this process may use (lscpu, else /proc/cpuinfo)."""
    info = {"model": None, "physical_cores": None}
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        kv = {ln.split(":", 1)[0].strip(): ln.split(":", 1)[1].strip() for ln in out.splitlines() if ":" in ln}
        info["model"] = kv.get("Model name")
        if kv.get("Core(s) per socket") and kv.get("Socket(s)"):
            info["physical_cores"] = int(kv["Core(s) per socket"]) * int(kv["Socket(s)"])
    except (OSError, subprocess.SubprocessError, ValueError):
        pass
    if info["model"] is None and os.path.exists("/proc/cpuinfo"):
        for ln in open("/proc/cpuinfo"):
            if ln.startswith("model name"):
                info["model"] = ln.split(":", 1)[1].strip()
                break
    avail = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    env = os.environ.get("OMP_NUM_THREADS")
    info["threads"] = min(avail, int(env)) if env and env.isdigit() and int(env) > 0 else avail
    info["logical_cpus_visible"] = avail
    return info


def profile_traffic(name: str):
    """Bytes per launch from a committed rocprofv3 PMC summary (FETCH_SIZE + WRITE_SIZE, copy-calibrated)."""
    path = os.path.join(ROOT, "profiles", name)
    if os.path.exists(path):
        for line in open(path):
            if line.startswith("traffic_bytes_per_launch:"):
                return float(line.split(":", 1)[1]), f"profiles/{name} (rocprofv3 --pmc, not measured in this run)"
    return None, None


def main() -> None:
    args = parse()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: the online-FP8 path runs on one GPU only (the full token sequence resident, no sharding, no "
              "collectives); --gpus must be 1", file=sys.stderr)
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

    def settle(fn, seconds=None):
        """Untimed calls for `seconds` (default --settle-s): the clock climbs back after the host-side set-up."""
        t_a = time.perf_counter()
        n = 0
        while time.perf_counter() - t_a < (args.settle_s if seconds is None else seconds) or n < 2:
            fn()
            n += 1
            if n % 16 == 0:
                torch.cuda.synchronize()
        torch.cuda.synchronize()

    def time_steps(fn, steps, warmup):
        """Total time of `steps` back-to-back calls (ms), after a clock settle and `warmup` untimed ones; synchronised
        on both sides."""
        settle(fn)
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

    def tflops(f, ms):
        return f / (ms * 1e-3) / 1e12

    def gbs(b, ms):
        return b / (ms * 1e-3) / 1e9

    out = {}

    if args.copy_calibration:
        src = torch.empty(512 << 20, device=dev, dtype=torch.uint8).fill_(1)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst

    # ---- headline: the block linear chain at 1344x768 15 s (M = 91 x 1008) ----
    c4 = synthetic.CONFIGS["c4_chain_1344x768_15s"]
    M, H, F = c4["M"], c4["K"], 8192
    x4 = synthetic.activations(M, H, seed=0, n_out=c4["n_out"]).to(dev)
    xo = synthetic.activations(M, H, seed=5, n_out=c4["n_out"]).to(dev)     # attention-output stand-in
    wqkv, sqkv = quantised_weight(3 * H, H, seed=1)
    wo, so = quantised_weight(H, H, seed=4)
    wgu, sgu = quantised_weight(2 * F, H, seed=2)
    wd, sd = quantised_weight(H, F, seed=3)
    E4 = ops.E4M3

    def buf(shape, dt):
        return torch.empty(shape, device=dev, dtype=dt)

    q0, s0 = buf((M, H), E4), buf((M, 1), torch.float32)
    yqkv = buf((M, 3 * H), torch.bfloat16)
    qo, s_o = buf((M, H), E4), buf((M, 1), torch.float32)
    y_out, amax_o = buf((M, H), torch.bfloat16), buf((M,), torch.float32)
    qg, sg = buf((M, H), E4), buf((M, 1), torch.float32)
    hws, amax_h = buf((M, F), torch.bfloat16), buf((M,), torch.float32)
    qh, sh = buf((M, F), E4), buf((M, 1), torch.float32)
    y_d, amax_d = buf((M, H), torch.bfloat16), buf((M,), torch.float32)
    qn, sn = buf((M, H), E4), buf((M, 1), torch.float32)

    # (name, launch, algorithmic FLOPs, algorithmic HBM bytes) of every kernel launch of one chain step, in order
    seg = [
        ("quant_x [M,3072] (kernel 1)", lambda: ops.quant_rows(x4, q0, s0), 0.0, 3.0 * M * H + 4 * M),
        ("qkv_gemm 3072->9216 (kernel 2)", lambda: ops.gemm(q0, wqkv, s0, sqkv, torch.bfloat16, out=yqkv),
         2.0 * M * 3 * H * H, 0.0),
        ("quant_attn [M,3072] (kernel 1)", lambda: ops.quant_rows(xo, qo, s_o), 0.0, 3.0 * M * H + 4 * M),
        ("out_gemm 3072->3072 + row amax (kernel 2)",
         lambda: ops.gemm(qo, wo, s_o, so, torch.bfloat16, out=y_out, row_amax=amax_o), 2.0 * M * H * H, 0.0),
        ("out quant tail [M,3072]", lambda: ops.quant_rows_amax(y_out, amax_o, qg, sg), 0.0, 3.0 * M * H + 4 * M),
        ("gate_up_swiglu 3072->2x8192 + row amax (kernel 3)",
         lambda: ops.gemm_swiglu(qg, wgu, sg, sgu, row_amax=amax_h, out=hws), 2.0 * M * 2 * F * H, 0.0),
        ("swiglu requant tail [M,8192]", lambda: ops.quant_rows_amax(hws, amax_h, qh, sh), 0.0, 3.0 * M * F + 4 * M),
        ("down_gemm 8192->3072 + row amax (kernel 2)",
         lambda: ops.gemm(qh, wd, sh, sd, torch.bfloat16, out=y_d, row_amax=amax_d), 2.0 * M * H * F, 0.0),
        ("down quant tail [M,3072]", lambda: ops.quant_rows_amax(y_d, amax_d, qn, sn), 0.0, 3.0 * M * H + 4 * M),
    ]
    IDX_K3 = 5                                               # kernel 3's launch in `seg`
    flops = sum(x[2] for x in seg)

    def chain_step(marks=None):
        for i, (_, fn, _, _) in enumerate(seg):
            if marks is not None:
                marks[i].record(stream)
            fn()
        if marks is not None:
            marks[len(seg)].record(stream)

    # clock pre-roll, then the warm-up steps, then the timed steps (no events inside: an event recorded between two
    # launches adds its own cost, a few us), then as many steps again with one event before every launch, for the
    # per-launch breakdown and the roofline
    t_pre = time.perf_counter()
    n_pre = 0
    while time.perf_counter() - t_pre < args.preroll_s or n_pre < 2:
        chain_step()
        n_pre += 1
        if n_pre % 8 == 0:
            torch.cuda.synchronize()
    torch.cuda.synchronize()
    preroll_ms = (time.perf_counter() - t_pre) * 1e3
    steps, warm = args.steps, args.warmup
    for _ in range(warm):
        chain_step()
    marks = [[ev() for _ in range(len(seg) + 1)] for _ in range(steps)]
    torch.cuda.synchronize()
    t0, t1 = ev(), ev()
    t0.record(stream)
    for k in range(steps):
        chain_step()
    t1.record(stream)
    t1.synchronize()
    torch.cuda.synchronize()
    t_step = t0.elapsed_time(t1) / steps
    value = tflops(flops, t_step)
    t0.record(stream)
    for k in range(steps):
        chain_step(marks[k])
    t1.record(stream)
    t1.synchronize()
    torch.cuda.synchronize()
    t_step_ev = t0.elapsed_time(t1) / steps
    seg_ms = [sum(marks[k][i].elapsed_time(marks[k][i + 1]) for k in range(steps)) / steps for i in range(len(seg))]
    breakdown = {}
    for (name, _, f, b), ms in zip(seg, seg_ms):
        e = {"ms": round(ms, 4)}
        if f:
            e["TFLOP/s"] = round(tflops(f, ms), 1)
            e["frac_mfma"] = round(tflops(f, ms) / PEAK_TFLOPS, 4)
        else:
            e["GB/s"] = round(gbs(b, ms), 1)
            e["frac_hbm"] = round(gbs(b, ms) / PEAK_GBS, 4)
        breakdown[name] = e
    gemm_ms = sum(ms for (_, _, f, _), ms in zip(seg, seg_ms) if f)
    k3_tf = tflops(seg[IDX_K3][2], seg_ms[IDX_K3])
    traffic, traffic_src = profile_traffic("gemm_swiglu_c4_1344x768_15s_traffic.txt")
    roofline = {"bound": "mfma", "achieved": round(k3_tf, 1), "peak": PEAK_TFLOPS, "unit": "TFLOP/s",
                "frac": round(k3_tf / PEAK_TFLOPS, 4), "traffic": traffic, "traffic_source": traffic_src,
                "kernel": "gemm_kernel<EPI_SWIGLU> (kernel 3: gate/up GEMM + SwiGLU epilogue + row amax), c4",
                "launch_ms": round(seg_ms[IDX_K3], 4), "flops_per_launch": seg[IDX_K3][2],
                "timing": f"HIP events around each of its {steps} launches in the steps timed with events, on the "
                          "launch stream (the row-amax zero-fill kernel before it included)"}
    c4_line = {"breakdown": breakdown,
               "gemms_TFLOP/s": round(tflops(flops, gemm_ms), 1),
               "gemms_frac_mfma": round(tflops(flops, gemm_ms) / PEAK_TFLOPS, 4),
               "sum_of_launches_ms": round(sum(seg_ms), 4),
               "step_with_events_ms": round(t_step_ev, 4),
               "step_minus_launches_ms": round(t_step_ev - sum(seg_ms), 4),
               "note": "out-proj input is a seeded bf16 stand-in for the attention output; value counts the four "
                       "GEMMs' FLOPs over the whole step (quant and tail passes included in the time)"}
    def want(name):
        return "none" not in only and (not only or name in only)

    if want("power"):
        # Socket power and gfx clock while each launch of the chain runs back to back for --power-s seconds, beside
        # the register-only MFMA loop (the chip's sustained FP8 MFMA rate with no memory traffic): the FP8 GEMMs run
        # at the 1400 W board limit, where the clock, not the schedule, sets the MFMA rate.
        import shutil
        import threading
        smi = shutil.which("amd-smi")
        if smi is None:
            out["power_clock"] = {"skipped": "amd-smi not found"}
        else:
            samples, stop = [], []

            def sampler():
                while not stop:
                    t_s = time.time()
                    try:
                        samples.append((t_s,) + smi_sample(smi))
                    except Exception:                   # a missed sample only thins the window
                        pass
                    time.sleep(0.2)

            ml_out = torch.empty(256 * 256, device=dev, dtype=torch.float32)
            ml_iters = 10000
            legs = [("mfma_register_loop (no memory traffic)", lambda: ops.mfma_loop(ml_out, ml_iters),
                     ops.MFMA_LOOP_FLOP_PER_ROUND * 256 * ml_iters, 0.0)]
            legs += [seg[i] for i in (1, 3, IDX_K3, 7, 0)]
            th = threading.Thread(target=sampler, daemon=True)
            th.start()
            pw = {}
            ceiling = None
            for name, fn, f, b in legs:
                fn()
                torch.cuda.synchronize()
                e0, e1 = ev(), ev()
                t_a = time.time()
                n = 0
                e0.record(stream)
                while time.time() - t_a < args.power_s:
                    for _ in range(4):
                        fn()
                    n += 4
                    torch.cuda.synchronize()
                e1.record(stream)
                e1.synchronize()
                t_b = time.time()
                ms = e0.elapsed_time(e1) / n
                win = sorted((p, c) for t_s, p, c in samples if t_a + 0.6 <= t_s <= t_b)
                e = {"ms": round(ms, 4), "samples": len(win)}
                if win:
                    e["socket_power_W"] = win[len(win) // 2][0]
                    e["gfx_clock_MHz"] = round(sorted(c for _, c in win)[len(win) // 2])
                if f:
                    e["TFLOP/s"] = round(tflops(f, ms), 1)
                    e["frac_mfma"] = round(tflops(f, ms) / PEAK_TFLOPS, 4)
                    if ceiling is None:
                        ceiling = tflops(f, ms)
                    else:
                        e["frac_of_register_loop"] = round(tflops(f, ms) / ceiling, 4)
                else:
                    e["GB/s"] = round(gbs(b, ms), 1)
                    e["frac_hbm"] = round(gbs(b, ms) / PEAK_GBS, 4)
                pw[name] = e
            stop.append(True)
            th.join()
            pw["note"] = ("median socket power and gfx clock (amd-smi, every ~0.3 s) over each back-to-back run after "
                          "its first 0.6 s; the 5.0 PFLOP/s peak is quoted at the 2.4 GHz maximum clock")
            out["power_clock"] = pw
            del ml_out
    del x4, xo, yqkv, hws, y_out, y_d, q0, qo, qg, qh, qn

    # ---- the other measured workloads ----

    if want("c2") or want("vendor"):
        # The QKV projection at the 5 s 960x576 token count (M = 31 x 540): quant of X + kernel 2, with the two
        # launches timed by events inside the timed steps (the gap between the step and its launches is what the
        # host's back-to-back launches leave between them).
        c2 = synthetic.CONFIGS["c2_qkv_960x576_5s"]
        M2, K2, N2 = c2["M"], c2["K"], c2["N"]
        x2 = synthetic.activations(M2, K2, seed=0, n_out=c2["n_out"]).to(dev)
        w2, sw2 = quantised_weight(N2, K2, seed=1)
        q2, sq2 = buf((M2, K2), E4), buf((M2, 1), torch.float32)
        y2 = buf((M2, N2), torch.bfloat16)
        f2 = 2.0 * M2 * N2 * K2
        ev2 = [[ev() for _ in range(3)] for _ in range(steps)]

        def c2_step(m=None):
            if m:
                m[0].record(stream)
            ops.quant_rows(x2, q2, sq2)
            if m:
                m[1].record(stream)
            ops.gemm(q2, w2, sq2, sw2, torch.bfloat16, out=y2)
            if m:
                m[2].record(stream)
        settle(c2_step)
        for _ in range(max(warm, 20)):
            c2_step()
        torch.cuda.synchronize()
        a0, a1 = ev(), ev()
        a0.record(stream)
        for k in range(steps):
            c2_step(ev2[k])
        a1.record(stream)
        a1.synchronize()
        t2 = a0.elapsed_time(a1) / steps
        tq2 = sum(e[0].elapsed_time(e[1]) for e in ev2) / steps
        tg2 = sum(e[1].elapsed_time(e[2]) for e in ev2) / steps
        qb2 = 3.0 * M2 * K2 + 4.0 * M2
        if want("c2"):
            # Events around a 23-26 us launch add their own cost to it (a kernel trace of these steps shows the quant
            # at 23.5-24.5 us where its events measure 27-31 us).  So the step and the quant's share of it are timed
            # without events inside: 12 rounds of 2 x steps whole steps, then as many GEMM calls alone; the quant's
            # figure is the median over the rounds of the time it adds to a step (its launch gap included).  The
            # quant alone, back to back, beside it.
            def block(fn, n):
                s_, e_ = ev(), ev()
                s_.record(stream)
                for _ in range(n):
                    fn()
                e_.record(stream)
                e_.synchronize()
                return s_.elapsed_time(e_) / n

            gemm_only = lambda: ops.gemm(q2, w2, sq2, sw2, torch.bfloat16, out=y2)  # noqa: E731
            settle(c2_step)
            rounds = [(block(c2_step, 2 * steps), block(gemm_only, 2 * steps)) for _ in range(12)]
            med = lambda v: sorted(v)[len(v) // 2]  # noqa: E731
            t2c, tgo = med([r[0] for r in rounds]), med([r[1] for r in rounds])
            tqs = med([r[0] - r[1] for r in rounds])
            tqb = time_steps(lambda: ops.quant_rows(x2, q2, sq2), 4 * steps, warm) / (4 * steps)
            out["c2_qkv_960x576_5s"] = {
                "ms_per_step": round(t2c, 4), "TFLOP/s": round(tflops(f2, t2c), 1),
                "kernel2_ms": round(tg2, 4), "kernel2_TFLOP/s": round(tflops(f2, tg2), 1),
                "kernel2_frac_mfma": round(tflops(f2, tg2) / PEAK_TFLOPS, 4),
                "kernel2_back_to_back_ms": round(tgo, 4),
                "quant_ms": round(tqs, 4), "quant_GB/s": round(gbs(qb2, tqs), 1),
                "quant_frac_hbm": round(gbs(qb2, tqs) / PEAK_GBS, 4),
                "quant_timing": "median over 12 rounds of the step's time minus the GEMM's time alone, both without "
                                "events inside",
                "quant_events_ms": round(tq2, 4),
                "quant_back_to_back": {"ms": round(tqb, 4), "GB/s": round(gbs(qb2, tqb), 1),
                                       "frac_hbm": round(gbs(qb2, tqb) / PEAK_GBS, 4)},
                "step_with_events_ms": round(t2, 4),
                "step_minus_launches_ms": round(t2 - tq2 - tg2, 4)}
        if want("vendor"):
            # The same GEMM through the vendor library (torch._scaled_mm -> hipBLASLt) on the same fp8 operands and
            # per-token / per-channel scales, bf16 out: the practical reference point for kernel 2 on this chip.
            try:
                sa2, sb2 = sq2.view(M2, 1), sw2.view(1, N2)
                t_v = time_steps(lambda: torch._scaled_mm(q2, w2.t(), sa2, sb2, out_dtype=torch.bfloat16), steps,
                                 warm) / steps
                one = torch.ones((), device=dev)
                t_vt = time_steps(lambda: torch._scaled_mm(q2, w2.t(), one, one, out_dtype=torch.bfloat16), steps,
                                  warm) / steps
                t_k2 = time_steps(lambda: ops.gemm(q2, w2, sq2, sw2, torch.bfloat16, out=y2), steps, warm) / steps
                out["vendor_gemm_qkv_960x576"] = {
                    "library": "torch._scaled_mm (hipBLASLt)",
                    "rowwise_scales_TFLOP/s": round(tflops(f2, t_v), 1),
                    "tensorwise_scales_TFLOP/s": round(tflops(f2, t_vt), 1),
                    "kernel2_TFLOP/s": round(tflops(f2, t_k2), 1)}
            except Exception as exc:  # noqa: BLE001
                out["vendor_gemm_qkv_960x576"] = {"error": f"{type(exc).__name__}: {str(exc)[:160]}"}
        del x2, w2, q2, y2

    if want("outq"):
        # The out projection's input quantised straight from a Ulysses reverse all-to-all's receive buffer
        # (h3_tp2/ulysses_outq.py:138-143): one GPU's share of the 1344x768 15 s chain on two ranks, recv [P = 2,
        # M / 2 = 45 864, 12 heads, 128], row m = recv[0, m] | recv[1, m]; beside kernel 1 on the unpacked rows.
        P, Ml, hl, hd = 2, synthetic.CONFIGS["c4_chain_1344x768_15s"]["M"] // 2, 12, 128
        Kq = P * hl * hd
        recv = (torch.randn(P, Ml, hl, hd, device=dev) * 2).to(torch.bfloat16)
        unp = recv.permute(1, 0, 2, 3).reshape(Ml, Kq).contiguous()
        qo, so = buf((Ml, Kq), E4), buf((Ml, 1), torch.float32)
        by_q = 3.0 * Ml * Kq + 4.0 * Ml
        t_seg = time_steps(lambda: ops.quant_from_recv(recv), steps, warm) / steps
        t_unp = time_steps(lambda: ops.quant_rows(unp, qo, so), steps, warm) / steps
        out[f"receive_buffer_quant_{P}x{Ml}x{hl}x{hd}"] = {
            "ms": round(t_seg, 4), "GB/s": round(gbs(by_q, t_seg), 1),
            "frac_hbm": round(gbs(by_q, t_seg) / PEAK_GBS, 4), "kernel1_on_unpacked_rows_ms": round(t_unp, 4),
            "form": "kernel 1 over the P row segments of the receive buffer (no unpack copy); 3 K + 4 bytes per row"}
        del recv, unp, qo, so

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
        out["c1_single_linear_2048x3072x3072"] = {
            "ms": round(t, 4), "TFLOP/s": round(2.0 * M1 * N1 * K1 / (t * 1e-3) / 1e12, 1),
            "frac_mfma": round(2.0 * M1 * N1 * K1 / (t * 1e-3) / 1e12 / PEAK_TFLOPS, 4),
            "form": "kernel 1 + kernel 2 as 256 tiles of 128 tokens x 192 weight rows, one per CU"}
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
        ya = torch.empty((Mg, Ng), device=dev, dtype=torch.bfloat16)
        t2_eager = time_steps(lambda: ops.gemm(qa, wa, sqa, swa, torch.bfloat16, out=ya), steps, warm) / steps
        # eager back-to-back calls are host-bound at this size (one Python call costs about as much as the kernel):
        # the kernel's rate comes from one HIP graph of `steps` calls, replayed
        g_ad = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g_ad):
            for _ in range(steps):
                ops.gemm(qa, wa, sqa, swa, torch.bfloat16, out=ya)
        t2 = time_steps(g_ad.replay, 3, 2) / 3 / steps
        del g_ad
        # the same calls rotating over 6 copies of the weight (340 MB, more than the 256 MB MALL), so that each call
        # reads its weight from HBM rather than from the MALL
        wcopies = [wa.clone() for _ in range(6)]
        g_cold = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g_cold):
            for i in range(steps):
                ops.gemm(qa, wcopies[i % 6], sqa, swa, torch.bfloat16, out=ya)
        t2_cold = time_steps(g_cold.replay, 3, 2) / 3 / steps
        del g_cold, wcopies
        wbytes = float(Ng * Kg)
        out["c5_grouped_one_launch"]["adaLN_M2_alone"] = {
            "ms": round(t2, 4), "GB/s": round(wbytes / (t2 * 1e-3) / 1e9, 1),
            "frac_hbm": round(wbytes / (t2 * 1e-3) / 1e9 / PEAK_GBS, 4),
            "weight_from_hbm": {"ms": round(t2_cold, 4), "GB/s": round(wbytes / (t2_cold * 1e-3) / 1e9, 1),
                                "frac_hbm": round(wbytes / (t2_cold * 1e-3) / 1e9 / PEAK_GBS, 4),
                                "note": "calls rotating over 6 weight copies (340 MB > the 256 MB MALL)"},
            "eager_calls_ms": round(t2_eager, 4),
            "timing": f"one HIP graph of {steps} calls, replayed (eager_calls_ms: back-to-back Python calls); the "
                      "weight stays in the MALL between these calls",
            "form": f"kernel 2's small-M form on [{Mg},{Kg}] x [{Ng},{Kg}]: {Ng // 16} waves of 16 weight rows, "
                    "the weight streamed once (output bitwise the tiled kernel's)"}
        del probs, xs

    if want("h3_linears"):
        # The reference's own H3 DiT linears at its published per-rank row count M = 42 848 (qkv 5376 -> 21 504, out
        # 7168 -> 5376, fc1 5376 -> 2 x 14 336 with the SwiGLU epilogue and the requant tail, fc2 14 336 -> 5376),
        # log-normal activation rows exp(N(0, 1) 1.5) (its probe inputs), each launch timed by events inside the timed
        # steps.
        Mh = 42848
        specs = [("qkv 5376->21504 (kernel 2)", 5376, 21504, False), ("out 7168->5376 (kernel 2)", 7168, 5376, False),
                 ("fc1 5376->2x14336 + SwiGLU + row amax (kernel 3)", 5376, 28672, True),
                 ("fc2 14336->5376 (kernel 2)", 14336, 5376, False)]
        launches = []
        genh = torch.Generator(device=dev).manual_seed(40)
        for i, (name, Kh, Nh, swiglu) in enumerate(specs):
            # made on the device (a timing workload; 0.6 G elements would take the host ~10 s)
            xh = (torch.randn(Mh, Kh, device=dev, generator=genh)
                  * torch.exp(torch.randn(Mh, 1, device=dev, generator=genh) * 1.5)).to(torch.bfloat16)
            ah, sah = ops.quant_rows(xh)
            del xh
            wh, swh = quantised_weight(Nh, Kh, seed=50 + i)
            if swiglu:
                hh, amh = buf((Mh, Nh // 2), torch.bfloat16), buf((Mh,), torch.float32)
                qhh, shh = buf((Mh, Nh // 2), E4), buf((Mh, 1), torch.float32)
                launches.append((name, (lambda a_=ah, w_=wh, s_=sah, t_=swh, h_=hh, m_=amh:
                                        ops.gemm_swiglu(a_, w_, s_, t_, row_amax=m_, out=h_)), 2.0 * Mh * Nh * Kh, 0.0))
                launches.append(("fc1 requant tail [M,14336]", (lambda h_=hh, m_=amh, q_=qhh, s_=shh:
                                                                ops.quant_rows_amax(h_, m_, q_, s_)),
                                 0.0, 3.0 * Mh * (Nh // 2) + 4.0 * Mh))
            else:
                yh = buf((Mh, Nh), torch.bfloat16)
                launches.append((name, (lambda a_=ah, w_=wh, s_=sah, t_=swh, y_=yh:
                                        ops.gemm(a_, w_, s_, t_, torch.bfloat16, out=y_)), 2.0 * Mh * Nh * Kh, 0.0))
        hsteps = max(5, steps // 3)
        settle(lambda: [fn() for _, fn, _, _ in launches])
        for _ in range(3):
            for _, fn, _, _ in launches:
                fn()
        hm = [[ev() for _ in range(len(launches) + 1)] for _ in range(hsteps)]
        torch.cuda.synchronize()
        for k in range(hsteps):
            for i, (_, fn, _, _) in enumerate(launches):
                hm[k][i].record(stream)
                fn()
            hm[k][-1].record(stream)
        hm[-1][-1].synchronize()
        lm = [sum(hm[k][i].elapsed_time(hm[k][i + 1]) for k in range(hsteps)) / hsteps for i in range(len(launches))]
        hres = {}
        for (name, _, f, b), ms in zip(launches, lm):
            hres[name] = ({"ms": round(ms, 4), "TFLOP/s": round(tflops(f, ms), 1),
                           "frac_mfma": round(tflops(f, ms) / PEAK_TFLOPS, 4)} if f else
                          {"ms": round(ms, 4), "GB/s": round(gbs(b, ms), 1), "frac_hbm": round(gbs(b, ms) / PEAK_GBS, 4)})
        fh = sum(f for _, _, f, _ in launches)
        gemm_h = sum(ms for (_, _, f, _), ms in zip(launches, lm) if f)
        out["h3_linears_42848"] = {
            "per_launch": hres, "step_ms": round(sum(lm), 4), "TFLOP/s": round(tflops(fh, sum(lm)), 1),
            "gemms_TFLOP/s": round(tflops(fh, gemm_h), 1), "gemms_frac_mfma": round(tflops(fh, gemm_h) / PEAK_TFLOPS, 4),
            "note": f"the reference's H3 linear shapes at its per-rank M = {Mh}; its published GB10 figures for the same "
                    "shapes (157-169 TFLOP/s per GEMM, another chip) are context, not a baseline"}
        del launches

    if want("dispatch"):
        # Host cost of one eligible call through the drop-in: vLLM's ops.cutlass_scaled_mm replaced by the dispatcher
        # (eligibility test -> route -> kernel 2's launcher -> ctypes -> the C ABI's launch), and QuantFP8.forward's
        # replacement on a dynamic per-token instance (-> kernel 1), on a small problem whose kernels take a few us,
        # so the host is the bound.  Wall time of 2000 back-to-back calls / 2000, with torch._scaled_mm (hipBLASLt) on
        # the same call for scale (the reference measures its dispatcher the same way against it).
        import types
        from h3_tp2_amd import fp8_gemm, fp8_quant_fuse
        Md, Nd, Kd = 32, 1024, 1024
        xd = synthetic.activations(Md, Kd, seed=60, n_out=1).to(dev)
        ad, sad = ops.quant_rows(xd)
        wd_, swd = quantised_weight(Nd, Kd, seed=61)
        bd = wd_.t()
        shim = types.SimpleNamespace(cutlass_scaled_mm=lambda *a, **k: None)
        saved_state = dict(fp8_gemm._state)
        fp8_gemm.install(shim, level="hip", check=False)
        qf = types.SimpleNamespace(static=False, use_per_token_if_dynamic=True, is_group_quant=False,
                                   num_token_padding=None)
        saved_k1 = fp8_quant_fuse._state.get("kernel1")
        fp8_quant_fuse._state["kernel1"] = True
        qfwd = fp8_quant_fuse.make_quant_forward(lambda self, x, *a, **k: None)

        def host_us(fn, n=2000):
            for _ in range(100):
                fn()
            torch.cuda.synchronize()
            t_a = time.perf_counter()
            for _ in range(n):
                fn()
            t_b = time.perf_counter()
            torch.cuda.synchronize()
            return (t_b - t_a) / n * 1e6
        sa2d, sb2d = sad.view(Md, 1), swd.view(1, Nd)
        res_d = {
            "shape": f"M={Md} N={Nd} K={Kd}",
            "dispatcher_cutlass_scaled_mm_us": round(host_us(lambda: shim.cutlass_scaled_mm(ad, bd, sad, swd,
                                                                                            torch.bfloat16)), 2),
            "ops_gemm_us": round(host_us(lambda: ops.gemm(ad, wd_, sad, swd)), 2),
            "torch_scaled_mm_us": round(host_us(lambda: torch._scaled_mm(ad, bd, sa2d, sb2d,
                                                                         out_dtype=torch.bfloat16)), 2),
            "quantfp8_forward_us": round(host_us(lambda: qfwd(qf, xd)), 2),
            "ops_quant_rows_us": round(host_us(lambda: ops.quant_rows(xd)), 2),
            "calls": 2000}
        # the same call with the block router in front of kernel 2 (fp8_cutlass.route's counterpart), inside a block's
        # routing scope that publishes the weight as the block's qkv weight: dispatcher -> router -> kernel 2
        from h3_tp2_amd import fp8_hip
        saved_routers, saved_hip = list(fp8_gemm._routers), dict(fp8_hip._state)
        fp8_hip._state.update(ok=True, reason="bench")
        fp8_gemm.set_router(fp8_hip.route)
        try:
            with fp8_hip._routing({fp8_hip.weight_key(bd): "qkv"}):
                res_d["dispatcher_with_block_router_us"] = round(
                    host_us(lambda: shim.cutlass_scaled_mm(ad, bd, sad, swd, torch.bfloat16)), 2)
        finally:
            fp8_gemm._routers[:] = saved_routers
            fp8_hip._state.clear()
            fp8_hip._state.update(saved_hip)
        out["dispatch_host_cost"] = res_d
        fp8_gemm._state.clear()
        fp8_gemm._state.update(saved_state)
        fp8_quant_fuse._state["kernel1"] = saved_k1

    if want("producers"):
        # The quant fused into its producers: norm1 + AdaLN -> QKV input at the 960x576 5 s token count, the gated
        # residual + norm2 + AdaLN -> fc1 input at the 1344x768 5 s count; H = 3072, a [6, 6H] modulation table.
        H = 3072
        M_qkv = synthetic.CONFIGS["c2_qkv_960x576_5s"]["M"]
        gen = torch.Generator(device=dev).manual_seed(7)
        res = {}
        for name, Mp, gate in (("qkv_rms_quant_16740x3072", M_qkv, False), ("fc1_gate_rms_quant_31248x3072",
                                                                         synthetic.CONFIGS["c3_ffn_1344x768_5s"]["M"],
                                                                         True)):
            xp = (torch.randn(Mp, H, device=dev, generator=gen)
                  * torch.exp(torch.randn(Mp, 1, device=dev, generator=gen))).to(torch.bfloat16)
            wn = (1.0 + 0.1 * torch.randn(H, device=dev, generator=gen)).to(torch.bfloat16)
            ada = torch.randn(6, 6 * H, device=dev, generator=gen).to(torch.bfloat16)
            shp, scp, gtp = ada[:, :H], ada[:, H:2 * H], ada[:, 2 * H:3 * H]
            # indices as the model forms them (one per timestep group and modality, so long runs of rows): the
            # first 540 rows (a conditioning span) on one index, the rest on another; and, for comparison with the
            # reference's producer probe (scripts/fp8_quant_fuse_probe.py:72), a random index per row
            idx = torch.zeros(Mp, dtype=torch.int64, device=dev)
            idx[:540] = 1
            idx_rand = torch.randint(0, 6, (Mp,), device=dev, generator=gen)
            if gate:
                br = torch.randn(Mp, H, device=dev, generator=gen).to(torch.bfloat16)
                fused = lambda: ops.gate_rms_quant(xp, gtp, br, wn, shp, scp, idx, 1e-6)  # noqa: E731
                fused_r = lambda: ops.gate_rms_quant(xp, gtp, br, wn, shp, scp, idx_rand, 1e-6)  # noqa: E731

                def unfused():
                    _, hh = ops.indexed_gate_rms_norm_scale_shift(xp, gtp, br, wn, shp, scp, idx, 1e-6)
                    ops.quant_rows(hh)
                nbytes = 7.0 * Mp * H + 4.0 * Mp          # residual, branch, residual_out (bf16) + q + scale
            else:
                fused = lambda: ops.rms_quant(xp, wn, shp, scp, idx, 1e-6)  # noqa: E731
                fused_r = lambda: ops.rms_quant(xp, wn, shp, scp, idx_rand, 1e-6)  # noqa: E731

                def unfused():
                    ops.quant_rows(ops.rms_norm_indexed_scale_shift(xp, wn, shp, scp, idx, 1e-6))
                nbytes = 3.0 * Mp * H + 4.0 * Mp          # x (bf16) + q + scale
            t_f = time_steps(fused, steps, warm) / steps
            t_r = time_steps(fused_r, steps, warm) / steps
            t_u = time_steps(unfused, steps, warm) / steps
            res[name] = {"ms": round(t_f, 4), "GB/s": round(nbytes / (t_f * 1e-3) / 1e9, 1),
                         "frac_hbm": round(nbytes / (t_f * 1e-3) / 1e9 / PEAK_GBS, 4),
                         "unfused_ms": round(t_u, 4), "speedup_vs_unfused": round(t_u / t_f, 3),
                         "indices": "runs (rows 0-539 one index, the rest another)",
                         "random_index_per_row": {"ms": round(t_r, 4),
                                                  "GB/s": round(nbytes / (t_r * 1e-3) / 1e9, 1),
                                                  "frac_hbm": round(nbytes / (t_r * 1e-3) / 1e9 / PEAK_GBS, 4)}}
            del xp, ada, idx, idx_rand
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
        T, Hq, N = synthetic.CONFIGS["c2_qkv_960x576_5s"]["M"], 3072 // 128, 9216
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
        # the plain scale pass of the two-pass form on the same product (bf16 out): the consumer every other site of
        # the two-pass level gets
        y_sp = torch.empty((T, N), device=dev, dtype=torch.bfloat16)
        t_sp = time_steps(lambda: ops.scale_bias_cast(x32, sa_t, sb_t, None, torch.bfloat16, out=y_sp), steps,
                          warm) / steps
        res["scale_pass_16740x9216"] = {"ms": round(t_sp, 4), "GB/s": round(qk_bytes / (t_sp * 1e-3) / 1e9, 1),
                                        "frac_hbm": round(qk_bytes / (t_sp * 1e-3) / 1e9 / PEAK_GBS, 4)}
        # the GEMM of the two-pass form: kernel 2 writing the raw fp32 product that the consumers above read (here
        # into the same buffer), QKV 3072 -> 9216 at 960x576 5 s
        qa, s_qa = ops.quant_rows(synthetic.activations(T, 3072, seed=11, n_out=3).to(dev))
        wq, s_wq = quantised_weight(N, 3072, seed=12)
        t_g32 = time_steps(lambda: ops.gemm(qa, wq, s_qa, s_wq, torch.float32, out=x32), steps, warm) / steps
        g32_flops = 2.0 * T * N * 3072
        res["two_pass_qkv_gemm_fp32_16740x9216x3072"] = {
            "ms": round(t_g32, 4), "TFLOP/s": round(tflops(g32_flops, t_g32), 1),
            "frac_mfma": round(tflops(g32_flops, t_g32) / PEAK_TFLOPS, 4),
            "with_qk_consumer_ms": round(t_g32 + t_qk, 4),
            "note": "kernel 2 storing the fp32 accumulator (2x the bf16 output bytes); with the fused qk consumer this is "
                    "the two-pass form of the QKV site"}
        del x32, st, y_sp, qa, wq
        Mc, H = synthetic.CONFIGS["c3_ffn_1344x768_5s"]["M"], 3072
        x32 = torch.randn(Mc, H, device=dev, generator=gen) * 3000
        sa_c = torch.rand(Mc, device=dev, generator=gen) * 1e-3 + 1e-4
        sb_c = torch.rand(H, device=dev, generator=gen) * 1e-3 + 1e-4
        resid = torch.randn(Mc, H, device=dev, generator=gen).to(torch.bfloat16)
        wn = (1.0 + 0.1 * torch.randn(H, device=dev, generator=gen)).to(torch.bfloat16)
        ada = torch.randn(6, 6 * H, device=dev, generator=gen).to(torch.bfloat16)
        # indices in runs as the model forms them, and a random index per row for comparison (see the producers)
        idx = torch.zeros(Mc, dtype=torch.int64, device=dev)
        idx[:540] = 1
        idx_rand = torch.randint(0, 6, (Mc,), device=dev, generator=gen)
        st = fc.Stash(x32, sa_c, sb_c, None, torch.empty((Mc, H), device=dev, dtype=torch.bfloat16))
        t_out = time_steps(lambda: fc.gate_rms_fused(st, resid, ada[:, 2 * H:3 * H], wn, ada[:, :H], ada[:, H:2 * H],
                                                     idx, 1e-6), steps, warm) / steps
        t_out_r = time_steps(lambda: fc.gate_rms_fused(st, resid, ada[:, 2 * H:3 * H], wn, ada[:, :H],
                                                       ada[:, H:2 * H], idx_rand, 1e-6), steps, warm) / steps
        out_bytes = Mc * H * (4.0 + 2 + 2 + 2)                       # product, residual in; residual_out, h out
        t_fc2 = time_steps(lambda: fc.gate_fused(st, resid, ada[:, 5 * H:], idx), steps, warm) / steps
        fc2_bytes = Mc * H * (4.0 + 2 + 2)                           # product, x in; out
        res["out_gate_rms_31248x3072"] = {"ms": round(t_out, 4), "GB/s": round(out_bytes / (t_out * 1e-3) / 1e9, 1),
                                          "frac_hbm": round(out_bytes / (t_out * 1e-3) / 1e9 / PEAK_GBS, 4),
                                          "indices": "runs (rows 0-539 one index, the rest another)",
                                          "random_index_per_row": {
                                              "ms": round(t_out_r, 4),
                                              "GB/s": round(out_bytes / (t_out_r * 1e-3) / 1e9, 1),
                                              "frac_hbm": round(out_bytes / (t_out_r * 1e-3) / 1e9 / PEAK_GBS, 4)}}
        res["fc2_indexed_gate_31248x3072"] = {"ms": round(t_fc2, 4),
                                              "GB/s": round(fc2_bytes / (t_fc2 * 1e-3) / 1e9, 1),
                                              "frac_hbm": round(fc2_bytes / (t_fc2 * 1e-3) / 1e9 / PEAK_GBS, 4)}
        del x32, st, resid, ada, idx, idx_rand
        # the fc1 stash forms of the two-pass MLP (1344x768 5 s, F = 8192): SwiGLU of the fp32 gate/up product to
        # bf16 h (level 1), and SwiGLU + per-token requant to e4m3 q + scale (level 2)
        F = 8192
        x32 = torch.randn(Mc, 2 * F, device=dev, generator=gen) * 3000
        sb_f = torch.rand(2 * F, device=dev, generator=gen) * 1e-3 + 1e-4
        t_sw = time_steps(lambda: ops.scale_swiglu(x32, sa_c, sb_f), steps, warm) / steps
        t_swq = time_steps(lambda: ops.scale_swiglu_quant(x32, sa_c, sb_f), steps, warm) / steps
        sw_bytes = Mc * F * (8.0 + 2)                                # gate + up fp32 in; h bf16 out
        swq_bytes = Mc * F * (8.0 + 1) + 4.0 * Mc                    # gate + up fp32 in; q + scale out
        res["fc1_scale_swiglu_31248x2x8192"] = {"ms": round(t_sw, 4),
                                                "GB/s": round(sw_bytes / (t_sw * 1e-3) / 1e9, 1),
                                                "frac_hbm": round(sw_bytes / (t_sw * 1e-3) / 1e9 / PEAK_GBS, 4)}
        res["fc1_scale_swiglu_quant_31248x2x8192"] = {"ms": round(t_swq, 4),
                                                      "GB/s": round(swq_bytes / (t_swq * 1e-3) / 1e9, 1),
                                                      "frac_hbm": round(swq_bytes / (t_swq * 1e-3) / 1e9 / PEAK_GBS,
                                                                        4)}
        del x32
        out["consumers_of_fp32_product"] = res

    # ---- CPU baseline: the reference's torch CPU path of the headline chain on a row sample ----
    cpu = None
    if not args.no_cpu:
        sys.path.insert(0, ROOT)
        from oracle import torch_path as TP
        hc = host_cpu()
        torch.set_num_threads(hc["threads"])
        rows = max(1, min(args.cpu_rows, M))
        xc = synthetic.activations(M, H, seed=0, n_out=c4["n_out"])[:rows]
        xoc = synthetic.activations(M, H, seed=5, n_out=c4["n_out"])[:rows]
        wts = {}
        for key, (n, k, seed) in {"qkv": (3 * H, H, 1), "out": (H, H, 4), "gate_up": (2 * F, H, 2),
                                  "down": (H, F, 3)}.items():
            wq_, sw_ = TP.quant(synthetic.weight(n, k, seed))
            wts[key] = (wq_, sw_.view(-1))
        TP.chain_step(xc[:64], xoc[:64], wts)                               # warm-up
        runs = []
        while len(runs) < 3 or sum(runs) < args.cpu_seconds:
            t_a = time.perf_counter()
            TP.chain_step(xc, xoc, wts)
            runs.append(time.perf_counter() - t_a)
        best = min(runs)
        f_rows = flops * rows / M
        cpu = {"value": round(f_rows / best / 1e12, 5), "unit": "TFLOP/s", "cores": hc["threads"], "kind": "port",
               "sample": f"the block chain (quant, fp32 torch matmul, epilogue; SwiGLU + requant) through the reference's "
                         f"torch CPU mirrors (oracle/torch_path.py) on the first {rows} of {M} token rows; min of "
                         f"{len(runs)} runs ({best:.2f} s; {sum(runs):.1f} s in all); the rate holds per row, so the "
                         f"full chain would take {best * M / rows:.1f} s",
               "cpu_model": hc["model"], "physical_cores": hc["physical_cores"],
               "logical_cpus_visible": hc["logical_cpus_visible"], "torch_threads": torch.get_num_threads()}

    line = {"metric": METRIC, "value": round(value, 1), "unit": "TFLOP/s", "n_gpus": 1, "steps": steps,
            "warmup": warm, "ms_per_step": round(t_step, 4), "higher_is_better": True, "scaling": "weak",
            "vs_baseline": None, "dtype": "e4m3", "data": "synthetic (seeded N(0,1) activations with x40 outlier "
            "channels, random-init N(0,0.02) weights)",
            "config": {"workload": "c4_chain_1344x768_15s: DiT block linear set QKV 3072->9216, out 3072->3072, "
                                   "gate/up 3072->2x8192 + SwiGLU, down 8192->3072, each input quantised per token "
                                   "(the next one fused into the previous epilogue)",
                       "M": M, "hidden": H, "ffn": F, "parallelism": "single GPU"},
            "preroll": {"ms": round(preroll_ms, 1), "chain_steps": n_pre},
            "roofline": roofline, "chain": c4_line, "cpu_baseline": cpu, "workloads": out}
    print(json.dumps(line))


if __name__ == "__main__":
    main()
