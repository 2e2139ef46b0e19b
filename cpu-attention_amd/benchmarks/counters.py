"""rocprofv3 columns for the benchmark rows (``bench.py --counters``).

For one row, the row's own arm runs again in child processes under rocprofv3
(``bench.py --profile-row NAME DTYPE ARM``: a 256 MiB device copy, then five calls
without cache flushes), one pass per counter set, since rocprofv3 collects a
limited number of counters per run:

* ``--kernel-trace``: device time of the library's kernels (names ``ca::...``)
  per call; a call's kernels are summed (a decode with a split combine, or a
  store before a decode, is two);
* ``--pmc FETCH_SIZE`` and ``--pmc WRITE_SIZE``: KiB read from and written to
  HBM per dispatch, each scaled by what the counter reads for the copy (whose
  bytes are known), summed over a call's kernels;
* ``--pmc MfmaUtil`` (prefill rows): rocprofv3's derived MFMA-busy percentage,
  MFMA-busy cycles over elapsed cycles times SIMDs.

The last call of each pass is reported (the earlier ones warm the caches and
the clock).  Every pass runs under a time limit of its own; a pass that fails
or finds no kernel leaves its column out.
"""

import csv
import glob
import os
import shutil
import subprocess
import sys
import tempfile

HERE = os.path.dirname(os.path.abspath(__file__))
COPY_BYTES = 256 << 20
CALLS = 5
PASS_TIMEOUT_S = 120


def _run(args, outdir):
    """One rocprofv3 pass over the profiled row; the CSV rows it wrote."""
    rocprof = shutil.which("rocprofv3")
    if rocprof is None:
        return None
    cmd = [rocprof, *args, "-d", outdir, "-o", "run", "--output-format", "csv", "--",
           sys.executable, os.path.join(HERE, "bench.py")]
    return cmd


def _csv(outdir, suffix):
    files = glob.glob(os.path.join(outdir, "**", f"*{suffix}"), recursive=True)
    if not files:
        return []
    with open(files[0]) as f:
        return list(csv.DictReader(f))


def dispatches(rows, value):
    """[(dispatch id, kernel name, value)] in dispatch order, one entry per
    dispatch (a counter reported per hardware instance is summed)."""
    per = {}
    for r in rows:
        d = int(r.get("Dispatch_Id") or r.get("Correlation_Id") or 0)
        v = value(r)
        if d in per:
            per[d] = (per[d][0], per[d][1] + v)
        else:
            per[d] = (r["Kernel_Name"], v)
    return [(d, n, v) for d, (n, v) in sorted(per.items())]


def last_call(entries):
    """(the calibration copy's value, the sum over the last call's library
    dispatches).  The copy is the largest device copy of the run (setup makes
    smaller ones) and runs right before the CALLS calls, whose dispatches come in
    equal groups; library dispatches before it belong to the row's setup (a
    decode row stages its cache through the API)."""
    copies = [(v, i) for i, (_, n, v) in enumerate(entries) if "copyBuffer" in n]
    if not copies:
        return None, None
    copy, at = max(copies)
    ours = [v for _, n, v in entries[at + 1:] if "ca::" in n]
    if not ours:
        return copy, None
    per_call = max(1, len(ours) // CALLS)
    return copy, sum(ours[-per_call:])


def parse_trace(rows):
    """Kernel-trace rows -> device µs of the last call's library kernels."""
    entries = dispatches(rows, lambda r: (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3)
    return last_call(entries)[1]


def parse_counter(rows, name, copy_bytes=COPY_BYTES):
    """--pmc rows of one counter -> bytes of the last call, scaled by the copy."""
    rows = [r for r in rows if r.get("Counter_Name") == name]
    copy, ours = last_call(dispatches(rows, lambda r: float(r["Counter_Value"])))
    if not copy or ours is None:
        return None
    return ours * copy_bytes / copy


def parse_util(rows):
    rows = [r for r in rows if r.get("Counter_Name") == "MfmaUtil"]
    entries = [(d, n, v) for d, n, v in dispatches(rows, lambda r: float(r["Counter_Value"])) if "ca::" in n]
    return entries[-1][2] if entries else None


def collect(name, dtype, arm, kind, table, host_checks="on"):
    """The counter columns of one row (missing ones left out)."""
    out = {}
    child = ["--profile-row", name, dtype, arm, "--table", table, "--host-checks", host_checks]
    passes = [("trace", ["--kernel-trace"]), ("fetch", ["--pmc", "FETCH_SIZE"]),
              ("write", ["--pmc", "WRITE_SIZE"])]
    if kind == "flash":
        passes.append(("util", ["--pmc", "MfmaUtil"]))
    env = dict(os.environ, TMPDIR=os.environ.get("TMPDIR", "/tmp"))
    for tag, opts in passes:
        with tempfile.TemporaryDirectory() as d:
            cmd = _run(opts, d)
            if cmd is None:
                return out
            try:
                r = subprocess.run([*cmd, *child], capture_output=True, text=True, timeout=PASS_TIMEOUT_S,
                                   env=env, cwd=d)
            except subprocess.TimeoutExpired:
                continue
            if "profiled" not in r.stdout:
                continue
            if tag == "trace":
                v = parse_trace(_csv(d, "kernel_trace.csv"))
                if v is not None:
                    out["kernel_us"] = v
            elif tag == "util":
                v = parse_util(_csv(d, "counter_collection.csv"))
                if v is not None:
                    out["mfma_util_pct"] = v
            else:
                v = parse_counter(_csv(d, "counter_collection.csv"), "FETCH_SIZE" if tag == "fetch" else "WRITE_SIZE")
                if v is not None:
                    out[f"{tag}_bytes"] = v
    if "fetch_bytes" in out and "write_bytes" in out:
        out["hbm_bytes"] = out["fetch_bytes"] + out["write_bytes"]
    return out
