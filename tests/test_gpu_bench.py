"""bench.py on the GPU: one short run keeps the one-JSON-line contract the benchmark driver reads
(required fields, the roofline and stage records, the secondary configurations)."""
import json
import subprocess
import sys

import pytest

import bench
from conftest import announce

pytestmark = pytest.mark.gpu


def test_bench_json_contract():
    announce("bench.py --steps 6 --warmup 2 --no-cpu-baseline")
    r = subprocess.run([sys.executable, "bench.py", "--steps", "6", "--warmup", "2",
                        "--no-cpu-baseline"], capture_output=True, text=True, cwd=bench.ROOT,
                       timeout=300)
    assert r.returncode == 0, r.stderr[-2000:]
    lines = [ln for ln in r.stdout.splitlines() if ln.strip()]
    assert len(lines) == 1
    d = json.loads(lines[0])
    for key in ("metric", "value", "unit", "n_gpus", "steps", "warmup", "ms_per_step",
                "higher_is_better", "scaling", "vs_baseline", "dtype", "data", "config",
                "roofline"):
        assert key in d, key
    assert d["metric"] == bench.METRIC and d["unit"] == "tokens/s" and d["n_gpus"] == 1
    assert d["steps"] == 6 and d["warmup"] == 2 and d["higher_is_better"] is True
    assert d["value"] > 0 and d["ms_per_step"] > 0
    assert abs(d["value"] - 4 * 4096 / (d["ms_per_step"] * 1e-3)) / d["value"] < 1e-3
    rf = d["roofline"]
    assert rf["bound"] == "hbm" and rf["unit"] == "GB/s" and rf["peak"] == 8000.0
    assert 0 < rf["frac"] < 1 and abs(rf["frac"] - rf["achieved"] / rf["peak"]) < 1e-3
    # achieved = the forward's compulsory bytes over the dominant kernel's event-timed duration
    assert rf["bytes"] == bench.compulsory_bytes(4, 16, 4096, 128, 128, 2)
    assert abs(rf["achieved"] - rf["bytes"] / (rf["kernel_avg_ms"] * 1e-3) / 1e9) / rf["achieved"] < 1e-3
    assert rf["traffic"] is None or rf["traffic"] > 0
    assert rf["device_copy_GBps"] > 0
    assert set(d["stages"]) == {"chunk_local", "scan_output"}
    assert set(d["secondary"]) == {"kda_config5", "gdn_config4_long_context",
                                   "kkt_inverse_config3", "deltanet_config1"}
    assert "cpu_baseline" not in d
