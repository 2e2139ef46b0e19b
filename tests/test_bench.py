"""bench.py's contract: one GPU only, traffic constants that agree with the committed
rocprof summaries, and (on a GPU) one JSON line with every field the driver reads."""

import json
import os
import re
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)


def run_bench(*args, timeout=600):
    return subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), *args], cwd=ROOT,
                          capture_output=True, text=True, timeout=timeout)


def test_more_than_one_gpu_exits_with_a_message():
    r = run_bench("--gpus", "2", timeout=300)
    assert r.returncode == 2
    assert "one GPU" in r.stderr


@pytest.mark.parametrize("name,profile", [
    ("decode", "decode_tiles_bf16_n64_h32_e128_p32.md"),
    ("prefill", "flash_bf16_causal_n4_l4096_h32_e128.md"),
])
def test_traffic_constants_match_the_profile_summaries(name, profile):
    """``roofline.traffic`` comes from the FETCH_SIZE/WRITE_SIZE figures the summary
    under profiles/ records; the two must not drift apart."""
    import bench
    text = open(os.path.join(ROOT, "profiles", profile)).read()
    stated = [int(m.replace(",", "")) for m in re.findall(r"KiB =\s+([\d,]+) B", text)]
    assert stated, "the summary states its traffic per call"
    assert bench.traffic_bytes(name) == stated[0]


@pytest.mark.gpu
def test_json_line_carries_the_contract(cuda):
    r = run_bench("--steps", "4", "--warmup", "4", "--no-cpu")
    assert r.returncode == 0, r.stderr[-2000:]
    lines = [ln for ln in r.stdout.splitlines() if ln.strip()]
    assert len(lines) == 1
    d = json.loads(lines[0])
    for key, kind in (("metric", str), ("value", float), ("unit", str), ("n_gpus", int), ("steps", int),
                      ("warmup", int), ("ms_per_step", float), ("higher_is_better", bool),
                      ("scaling", str), ("dtype", str), ("data", str), ("config", dict)):
        assert isinstance(d[key], kind), key
    assert (d["n_gpus"], d["steps"], d["warmup"]) == (1, 4, 4)
    assert d["vs_baseline"] is None and d["value"] > 0 and "workload" in d["config"]
    for roof in (d["roofline"], d["prefill"]["roofline"]):
        assert set(roof) >= {"bound", "achieved", "peak", "unit", "frac", "traffic"}
        assert 0 < roof["frac"] < 1 and roof["traffic"] > 0
        assert abs(roof["frac"] - roof["achieved"] / roof["peak"]) < 1e-3
    assert d["roofline"]["bound"] == "hbm" and d["prefill"]["roofline"]["bound"] == "mfma"
    assert d["us_per_call_cold"] > 0 and d["prefill"]["us_per_call_cold"] > 0
    # the clock ramp runs before the W warm-up calls of each leg, and is reported
    assert d["clock_ramp_calls"] > 0 and d["prefill"]["clock_ramp_calls"] > 0
    # every other BASELINE config, with its work, timings and roofline fraction
    cfgs = d["configs"]
    assert set(cfgs) == {"cfg1", "cfg2", "cfg4_cross", "cfg5_store", "cfg5_step"}
    for name, c in cfgs.items():
        assert c["value"] > 0 and 0 < c["roofline"]["frac"] < 1, name
        assert "algorithmic_bytes" in c or "algorithmic_flop" in c or "algorithmic_bytes_per_step" in c
    for name in ("cfg1", "cfg2", "cfg4_cross", "cfg5_store"):
        c = cfgs[name]
        assert c["us_per_call"] > 0 and c["us_per_call_cold"] > 0 and c["api_us_per_call"] > 0, name
    assert cfgs["cfg5_step"]["us_per_step"] > 0
