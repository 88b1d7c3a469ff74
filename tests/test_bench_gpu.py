"""bench.py's JSON line on the GPU: one short run of the default workload
through the product path, every field the driver reads present and consistent."""
import json
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.mark.gpu
def test_bench_line_contract():
    with open(os.path.join(ROOT, "BASELINE.json")) as f:
        metric = json.load(f)["metric"]
    cmd = [sys.executable, "-u", os.path.join(ROOT, "bench.py"), "--steps", "4", "--warmup", "2",
           "--cpu-runs", "1"]
    print("[case] bench.py --steps 4 --warmup 2 --cpu-runs 1", flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True, timeout=280, cwd=ROOT)
    assert r.returncode == 0, r.stderr[-2000:]
    lines = [ln for ln in r.stdout.splitlines() if ln.strip()]
    assert len(lines) == 1, lines
    d = json.loads(lines[0])
    assert d["metric"] == metric
    assert d["unit"] == "TFLOP/s" and d["higher_is_better"] is True and d["scaling"] == "weak"
    assert d["n_gpus"] == 1 and d["steps"] == 4 and d["warmup"] == 2
    assert d["vs_baseline"] is None and d["dtype"] == "f16" and d["data"].startswith("synthetic")
    assert d["config"]["workload"].startswith("cfg3") and "model" not in d["config"]
    assert (d["config"]["B"], d["config"]["S"], d["config"]["Hq"], d["config"]["D"]) == (4, 2048, 16, 128)
    # value: algorithmic fwd+bwd FLOPs of the step over its time
    flops = 3.5 * 4.0 * 4 * 16 * 2048 * 2048 * 128 / 2
    assert d["value"] == pytest.approx(flops / (d["ms_per_step"] * 1e-3) / 1e12, rel=2e-3)
    assert 0 < d["value"] < 2516.6
    ro = d["roofline"]
    assert ro["bound"] == "mfma" and ro["unit"] == "TFLOP/s" and ro["peak"] == 2516.6
    assert ro["frac"] == pytest.approx(ro["achieved"] / ro["peak"], rel=2e-3)
    assert ro["kernel"] in d["kernels"] and isinstance(ro["traffic"], (int, float))
    assert "profiles/attn_cfg3_traffic.md" in ro["traffic_source"]
    assert d["kernel_path"] == {"attn_fwd": ["fwd_asm"], "bwd_dq": ["dq_asm"], "bwd_dkdv": ["dkdv_asm"]}
    # cold cache: a separate figure after the timed region, never the value
    cc = d["cold_cache"]
    assert cc["flush_mib"] == 512 and cc["ms_per_step"] > 0 and cc["flush_ms"] > 0
    assert cc["tflops"] == pytest.approx(flops / (cc["ms_per_step"] * 1e-3) / 1e12, rel=2e-3)
    cb = d["cpu_baseline"]
    assert cb["kind"] == "port" and cb["unit"] == "TFLOP/s" and cb["value"] > 0
    assert 1 <= cb["cores"] <= 16 and cb["sample"]
