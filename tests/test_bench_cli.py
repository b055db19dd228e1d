"""bench.py's command line on the CPU: it refuses more than one GPU with a message (this path runs on one GPU; no
collectives) before it touches torch or a device."""
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                       timeout=60)
    assert r.returncode == 2
    assert "one GPU" in r.stderr and r.stdout == ""


def test_world_size_above_one_is_refused():
    env = dict(os.environ, WORLD_SIZE="2")
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py")], capture_output=True, text=True, timeout=60,
                       env=env)
    assert r.returncode == 2 and r.stdout == ""


def test_smi_sample_reads_socket_power_and_mean_gfx_clock(monkeypatch):
    """The power workload's sampler takes GPU 0's socket power and the mean of the per-XCD gfx clocks from
    `amd-smi metric -p -c --json` (the layout amd-smi 26 prints), skipping clock entries without a reading."""
    import importlib.util
    import json
    import types
    spec = importlib.util.spec_from_file_location("bench_mod", os.path.join(ROOT, "bench.py"))
    bench = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(bench)
    clocks = {f"gfx_{i}": {"clk": {"value": 1700 + 10 * i, "unit": "MHz"}} for i in range(8)}
    clocks["mem_0"] = {"clk": {"value": 2000, "unit": "MHz"}}
    clocks["gfx_8"] = {"clk": "N/A"}
    payload = {"gpu_data": [{"gpu": 0, "power": {"socket_power": {"value": 1400, "unit": "W"}}, "clock": clocks}]}
    seen = []

    def fake_run(cmd, **kw):
        seen.append(cmd)
        return types.SimpleNamespace(stdout=json.dumps(payload), returncode=0)

    monkeypatch.setattr(bench.subprocess, "run", fake_run)
    power, clk = bench.smi_sample("amd-smi")
    assert seen == [["amd-smi", "metric", "-p", "-c", "--json"]]
    assert power == 1400.0 and clk == sum(1700 + 10 * i for i in range(8)) / 8
