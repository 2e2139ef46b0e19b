"""The GPU benchmark harness (cpu-attention_amd/benchmarks): its rocprof counter
parsing on synthetic rocprofv3 CSV rows (CPU), and one small row end to end with
its JSON (GPU)."""

import json
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BENCH = os.path.join(ROOT, "cpu-attention_amd", "benchmarks")


def _counters():
    """The harness's counters module, loaded by path (the harness directory also
    holds a bench.py, which must not shadow the repository's own)."""
    import importlib.util
    spec = importlib.util.spec_from_file_location("harness_counters", os.path.join(BENCH, "counters.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def _trace_row(d, name, t0, t1):
    return {"Dispatch_Id": str(d), "Kernel_Name": name, "Start_Timestamp": str(t0), "End_Timestamp": str(t1)}


def _pmc_row(d, name, counter, value):
    return {"Dispatch_Id": str(d), "Kernel_Name": name, "Counter_Name": counter, "Counter_Value": str(value)}


def test_counter_parsing():
    counters = _counters()
    # setup (a staging call of the library, a small copy), the calibration copy,
    # then 5 calls of two kernels each
    rows = [_trace_row(0, "void ca::store_kernel<64>(ca::StoreParams)", 0, 99000),
            _trace_row(1, "__amd_rocclr_copyBuffer", 0, 1000),
            _trace_row(2, "__amd_rocclr_copyBuffer", 0, 90000)]
    d = 3
    for call in range(counters.CALLS):
        rows.append(_trace_row(d, "void ca::store_kernel<64>(ca::StoreParams)", 0, 5000 + call))
        rows.append(_trace_row(d + 1, "void ca::decode_tiles_kernel<128, true, false>(ca::DecodeParams)", 0, 20000))
        d += 2
    assert counters.parse_trace(rows) == pytest.approx((5004 + 20000) / 1e3)
    # FETCH_SIZE reported per hardware instance (two rows per dispatch), scaled by
    # the largest copy: the copy reads half its bytes on the counter
    kib = counters.COPY_BYTES / 1024 / 2
    pmc = [_pmc_row(1, "__amd_rocclr_copyBuffer", "FETCH_SIZE", 8.0),
           _pmc_row(2, "__amd_rocclr_copyBuffer", "FETCH_SIZE", kib / 2),
           _pmc_row(2, "__amd_rocclr_copyBuffer", "FETCH_SIZE", kib / 2)]
    for call in range(counters.CALLS):
        pmc.append(_pmc_row(10 + call, "void ca::flash_bf16_p64_kernel<128>(ca::FlashParams)", "FETCH_SIZE", 1000.0))
    assert counters.parse_counter(pmc, "FETCH_SIZE") == pytest.approx(1000.0 * 1024 * 2)
    util = [_pmc_row(10 + c, "void ca::flash_bf16_p64_kernel<128>(ca::FlashParams)", "MfmaUtil", 40.0 + c)
            for c in range(counters.CALLS)]
    assert counters.parse_util(util) == 44.0
    assert counters.parse_counter([], "WRITE_SIZE") is None


@pytest.mark.gpu
def test_one_row_end_to_end(cuda, tmp_path):
    out = tmp_path / "row.json"
    r = subprocess.run([sys.executable, os.path.join(BENCH, "bench.py"), "--json", str(out), "--table", "reference",
                        "--only", "N=1 L=128 S=128 H=16 E=64", "--dtype", "bf16"],
                       capture_output=True, text=True, timeout=300, cwd=ROOT)
    assert r.returncode == 0, r.stderr[-2000:]
    data = json.loads(out.read_text())
    assert "gfx950" in data["environment"]["library"] and data["environment"]["host_cores"] >= 1
    (row,) = data["rows"]
    assert row["kind"] == "flash" and row["dtype"] == "bf16" and row["ours"] == "ours"
    t = row["timing"]["ours"]
    assert 0 < t["gpu"]["median"] <= t["gpu"]["max"] and len(t["gpu"]["samples"]) == 10
    assert 0 < row["roofline"]["frac"] < 1 and row["tflops"] > 0
    # the comparator (torch SDPA's fused kernels) agrees with ours
    if row.get("ref"):
        assert row["max_diff"] < 5e-2


@pytest.mark.gpu
@pytest.mark.timeout(900)
def test_one_row_with_counters(cuda, tmp_path):
    """The same row with --counters: its rocprofv3 passes (kernel trace, FETCH_SIZE,
    WRITE_SIZE, MfmaUtil) run in child processes, and every column they add is
    there and consistent with the row: device time within the event-timed call,
    HBM bytes between half and ten times the row's algorithmic bytes (q, k, v
    read and out written once), the sum of fetch and write, and an MFMA-busy
    percentage in (0, 100]."""
    import shutil
    if shutil.which("rocprofv3") is None:
        pytest.skip("rocprofv3 is not on PATH")
    out = tmp_path / "row.json"
    print("harness row with --counters", flush=True)
    r = subprocess.run([sys.executable, os.path.join(BENCH, "bench.py"), "--json", str(out), "--table", "reference",
                        "--only", "N=1 L=128 S=128 H=16 E=64", "--dtype", "bf16", "--counters"],
                       capture_output=True, text=True, timeout=800, cwd=ROOT, env=dict(os.environ, TMPDIR="/tmp"))
    assert r.returncode == 0, r.stderr[-2000:]
    (row,) = json.loads(out.read_text())["rows"]
    c = row["counters"]
    assert set(c) >= {"kernel_us", "fetch_bytes", "write_bytes", "hbm_bytes", "mfma_util_pct"}, (c, r.stdout[-2000:])
    assert 0 < c["kernel_us"] <= row["timing"]["ours"]["gpu"]["max"]
    io = 1 * 128 * 16 * 64 * 2  # one of q, k, v, out in bf16
    assert 0.5 * 3 * io <= c["fetch_bytes"] <= 10 * 3 * io
    assert 0.5 * io <= c["write_bytes"] <= 10 * io
    assert c["hbm_bytes"] == pytest.approx(c["fetch_bytes"] + c["write_bytes"])
    assert 0 < c["mfma_util_pct"] <= 100
