"""bench.py's output contract, checked without a GPU: the one-GPU guard, and the committed
bench line (profiles/bench_line_default.json) against BASELINE.json's metric, the roofline
arithmetic and the committed traffic measurement."""
import json
import os
import subprocess
import sys

from conftest import ROOT


def test_bench_refuses_more_than_one_gpu():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 2
    msg = json.loads(r.stdout.strip().splitlines()[-1])
    assert "one GPU" in msg["error"]


def test_committed_bench_line_keeps_the_contract():
    line = json.load(open(os.path.join(ROOT, "profiles", "bench_line_default.json")))
    base = json.load(open(os.path.join(ROOT, "BASELINE.json")))
    assert line["metric"] == base["metric"]
    for k in ("value", "unit", "n_gpus", "steps", "warmup", "ms_per_step", "higher_is_better",
              "scaling", "vs_baseline", "dtype", "data", "config", "roofline", "cpu_baseline"):
        assert k in line, k
    assert line["n_gpus"] == 1 and line["vs_baseline"] is None and line["unit"] == "GB/s"
    assert "workload" in line["config"] and "model" not in line["config"]
    # value = the layer's algorithmic bytes / the layer time (layer_us is printed to
    # 0.01 us, which moves the quotient by up to ~3e-5 of itself)
    cfg = line["config"]
    assert abs(cfg["algorithmic_bytes"] / (cfg["layer_us"] * 1e3) - line["value"]) \
        <= 1e-4 * line["value"]
    roof = line["roofline"]
    assert roof["bound"] == "hbm" and roof["peak"] == 8000.0 and roof["unit"] == "GB/s"
    assert abs(roof["achieved"] / roof["peak"] - roof["frac"]) < 1e-4
    # launch_us is rounded to 0.01 us in the line: about 0.5 GB/s of slack at 120 us
    assert abs(roof["algorithmic_bytes_per_launch"] / (roof["launch_us"] * 1e3)
               - roof["achieved"]) < 1.0
    traffic = json.load(open(os.path.join(ROOT, "profiles", "traffic_wna16_w13_c3.json")))
    assert abs(roof["traffic"] - traffic["hbm_bytes_per_launch"]) <= 0.01 * roof["traffic"]
    att = roof["attainable_read"]
    assert abs(roof["achieved"] / att["value"] - roof["frac_of_attainable"]) < 1e-3
    pre = line["roofline_prefill"]
    assert pre["bound"] == "mfma" and pre["peak"] == 2500.0
    assert abs(pre["achieved"] / pre["peak"] - pre["frac"]) < 1e-4
    cpu = line["cpu_baseline"]
    for k in ("value", "unit", "cores", "kind", "sample"):
        assert k in cpu, k
    assert cpu["kind"] in ("port", "reference")
