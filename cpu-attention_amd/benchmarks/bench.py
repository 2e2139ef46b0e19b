"""Wall clock and device time of the MI355X build at its Python API, on the
reference's benchmark shapes and on the BASELINE configs.

    python cpu-attention_amd/benchmarks/bench.py --json out.json [--table reference|baseline|both]
        [--only 'N=8 '] [--dtype bf16|fp32|both]
    python cpu-attention_amd/benchmarks/report.py out.json    # markdown tables

Method (the reference's benchmarks/bench.py, moved to a GPU):

* Every arm is timed at its Python API, one call per sample, as a user calls it:
  ``flash_attn_func`` against torch's ``scaled_dot_product_attention`` (its fused
  flash / memory-efficient kernels on ROCm; the math fallback is never used) for
  prefill, and ``flash_attn_with_kvcache`` for paged decode (the reference's vLLM
  comparator has no GPU build here, so decode rows report the GPU's own
  bandwidth against the HBM roofline instead of a ratio).
* 3 warmup calls, then 10 timed calls per arm, interleaved across arms in a rotated
  order; before every call the GPU's caches are flushed by a write sweep over
  1 GiB (twice the 256 MB MALL plus the eight 4 MB L2s, with room to spare).
* Each sample records the API wall clock (host clock around the call, with the
  stream synchronised before and after) and the device time (HIP events recorded
  on the call's stream just before and after it; for calls shorter than their
  own host-side launch work this includes the host's gaps).  Medians decide; min
  and max are reported.
* ``--host-checks on`` (the default, as a user calls it) keeps the data-dependent
  ValueError checks, which read the index tensors on the host: one device
  synchronisation per decode or store call.  ``off`` is the serving setting
  (``CPU_ATTENTION_HOST_CHECKS=0``); the kernels stay in bounds either way.
* Paged rows run at page sizes 16 and 32 and keep the best, as the reference does.
* ``--counters`` adds rocprofv3 columns to every row: the row's own arm runs
  again, five calls without flushes, in a child process under ``rocprofv3``
  (``counters.py``): a kernel trace (device time of the library's kernels per
  call), ``FETCH_SIZE`` and ``WRITE_SIZE`` (HBM bytes per call, each scaled by
  what the counter reads for a 256 MiB copy in the same process), and for
  prefill rows ``MfmaUtil`` (MFMA-busy cycles over elapsed cycles).  The last
  call of each pass is the one reported.
* Rooflines: HBM 8 TB/s, dense MFMA 2.5 PFLOP/s bf16 and 157.3 TFLOP/s fp32.
  Decode bytes are the algorithmic ones (K and V of every visible token once, q,
  out, the new token's K/V read and written, page-table entries and lengths);
  prefill FLOP are 4*E per visible (query, key) pair.
"""

import argparse
import json
import os
import platform
import subprocess
import sys
import time

import numpy as np
import torch
import torch.nn.functional as F

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))  # cpu-attention_amd: the package
sys.path.insert(0, HERE)
import cpu_attention  # noqa: E402
from cpu_attention import _kernel  # noqa: E402
from report import label  # noqa: E402

DT = {"bf16": torch.bfloat16, "fp32": torch.float32}
WARMUP, RUNS, PAGES = 3, 10, (16, 32)
HBM_GBS, MFMA_TFLOPS = 8000.0, {"bf16": 2500.0, "fp32": 157.3}
FLUSH_BYTES = 1 << 30

# The reference's shape tables (benchmarks/bench.py:47-69), MHA.
# Prefill: (N, L = S, H, E, causal).
FLASH = [
    (1, 128, 16, 64, True),
    (1, 1024, 16, 64, True),
    (1, 2048, 32, 128, True),
    (1, 4096, 32, 128, True),
    (8, 512, 16, 64, False),
    (1, 1500, 20, 64, False),
    (8, 256, 16, 32, False),
]
# Paged decode, L = 1: (N, S, H, E, append); S a length or per-sequence lengths.
PAGED = [
    (1, 256, 16, 64, True),
    (1, 4096, 32, 128, True),
    (8, 1024, 16, 64, True),
    (8, 1024, 16, 32, True),
    (8, 4096, 32, 128, True),
    (8, [17, 255, 1023, 1025, 33, 513, 2047, 64], 16, 64, True),
    (8, 1500, 20, 64, False),
    (32, 512, 16, 64, True),
    (32, 1024, 32, 128, True),
]


def sh(*cmd):
    try:
        return subprocess.run(cmd, capture_output=True, text=True, timeout=20).stdout.strip()
    except Exception:  # noqa: BLE001
        return ""


class Flusher:
    """A write sweep over FLUSH_BYTES of device memory."""

    def __init__(self, dev):
        self.buf = torch.zeros(FLUSH_BYTES // 4, dtype=torch.int32, device=dev)

    def __call__(self):
        self.buf.add_(1)


PROFILE = {}  # --profile-row: the row and arm whose calls a rocprofv3 child records


class Profiled(Exception):
    """Raised once the profiled row's calls are done (nothing else runs)."""


def profile_calls(fn, calls=5):
    """The counters' calibration copy (256 MiB), then `calls` calls of `fn`."""
    src = torch.ones(64 << 20, dtype=torch.float32, device="cuda")
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    dst.copy_(src)
    torch.cuda.synchronize()
    del src, dst
    for _ in range(calls):
        fn()
    torch.cuda.synchronize()


def measure(fns, flush, row=None):
    """3 warmup + 10 timed calls per arm, rotated, caches flushed before each call.
    Returns per arm: API wall clock and device time (µs): median, min, max.
    In --profile-row mode, runs the chosen row's arm for rocprofv3 instead (and
    returns None for every other row); `row` is (name, dtype)."""
    if PROFILE:
        if row is not None and row != (PROFILE["row"], PROFILE["dtype"]):
            return None
        arm = PROFILE["arm"] if PROFILE["arm"] in fns else sorted(fns)[0]
        profile_calls(fns[arm])
        raise Profiled()
    names = list(fns)
    for n in names:
        for _ in range(WARMUP):
            flush()
            fns[n]()
    torch.cuda.synchronize()
    api = {n: [] for n in names}
    gpu = {n: [] for n in names}
    for r in range(RUNS):
        for n in names[r % len(names):] + names[:r % len(names)]:
            flush()
            torch.cuda.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            t0 = time.perf_counter_ns()
            e0.record()
            fns[n]()
            e1.record()
            torch.cuda.synchronize()
            api[n].append((time.perf_counter_ns() - t0) / 1000)
            gpu[n].append(e0.elapsed_time(e1) * 1000)

    def stats(x):
        return dict(median=float(np.median(x)), min=min(x), max=max(x), samples=x)

    return {n: dict(api=stats(api[n]), gpu=stats(gpu[n])) for n in names}


def flash_flop(n, l, s, h, e, causal):
    if not causal:
        return 4.0 * n * h * e * l * s
    vis = sum(max(0, min(s, i + 1 + s - l)) for i in range(l))
    return 4.0 * n * h * e * vis


def sdpa_arm(q, k, v, causal, out):
    """torch's fused SDPA kernels only (flash or memory-efficient); None when neither
    takes the call (the math fallback is never timed)."""
    from torch.nn.attention import SDPBackend, sdpa_kernel

    qt, kt, vt = (x.transpose(1, 2) for x in (q, k, v))

    def f():
        with sdpa_kernel([SDPBackend.FLASH_ATTENTION, SDPBackend.EFFICIENT_ATTENTION]):
            out["sdpa"] = F.scaled_dot_product_attention(qt, kt, vt, is_causal=causal).transpose(1, 2)
    try:
        f()
        torch.cuda.synchronize()
    except RuntimeError:
        return None
    return f


def flash_row(spec, dtype, dev, qkv_fused=False):
    b, s, h, d, causal = spec[:5]
    lq = spec[5] if len(spec) > 5 else s
    if qkv_fused:
        qkv = torch.randn(b * s, 3 * h * d, device=dev).to(dtype)
        q, k, v = (qkv[:, i * h * d:(i + 1) * h * d].view(b, s, h, d) for i in range(3))
    else:
        q = torch.randn(b, lq, h, d, device=dev).to(dtype)
        k, v = (torch.randn(b, s, h, d, device=dev).to(dtype) for _ in range(2))
    out = {}
    fns = {"ours": lambda: out.__setitem__("ours", cpu_attention.flash_attn_func(q, k, v, causal=causal))}
    if lq == s:
        f = sdpa_arm(q, k, v, causal, out)
        if f is not None:
            fns["sdpa"] = f
    esize = 2 if dtype == torch.bfloat16 else 4
    nbytes = (2 * b * lq * h * d + 2 * b * s * h * d) * esize  # q, out, k, v once each
    return fns, out, "sdpa", (flash_flop(b, lq, s, h, d, causal), nbytes)


def stage_cache(tokens, room, h, d, page, dtype, dev, seed=0):
    """Caches holding tokens[i] N(0,1) tokens per sequence, with pages for room[i]
    tokens, staged through the API (one prompt append per sequence, as the
    reference's benchmark does)."""
    g = torch.Generator(device=dev).manual_seed(seed)
    nb = [-(-n // page) for n in room]
    bt = torch.zeros(len(room), max(max(nb), 1), dtype=torch.int32)
    for i, n in enumerate(nb):
        bt[i, :n] = torch.arange(sum(nb[:i]), sum(nb[:i]) + n, dtype=torch.int32)
    bt = bt.to(dev)
    kc = torch.zeros(max(sum(nb), 1), h, page, d, dtype=dtype, device=dev)
    vc = torch.zeros_like(kc)
    q1 = torch.zeros(1, 1, h, d, dtype=dtype, device=dev)
    for i, n in enumerate(tokens):
        if n:
            k, v = (torch.randn(1, n, h, d, generator=g, device=dev).to(dtype) for _ in range(2))
            cpu_attention.flash_attn_with_kvcache(q1, kc, vc, k=k, v=v, cache_seqlens=0, page_table=bt[i:i + 1])
    return kc, vc, bt


def decode_bytes(lens, h, d, esize, append, width_used):
    kv = sum(2 * n * h * d * esize for n in lens)
    io = 2 * len(lens) * h * d * esize + width_used * 4 + len(lens) * 4
    if append:
        io += 2 * 2 * len(lens) * h * d * esize  # the new token's K/V read, then written
    return kv + io


def paged_row(spec, dtype, dev):
    b, ctx, h, d, append = spec
    lens = ctx if isinstance(ctx, list) else [ctx] * b
    staged = [n - 1 if append else n for n in lens]
    q = torch.randn(b, 1, h, d, device=dev).to(dtype)
    kn, vn = (torch.randn(b, 1, h, d, device=dev).to(dtype) for _ in range(2))
    before = torch.tensor(staged, dtype=torch.int32, device=dev)
    out, fns = {}, {}
    for page in PAGES:
        kc, vc, bt = stage_cache(staged, lens, h, d, page, dtype, dev)
        arm = f"ours p{page}"
        extra = dict(k=kn, v=vn) if append else {}
        fns[arm] = (lambda kc=kc, vc=vc, bt=bt, arm=arm, extra=extra: out.__setitem__(
            arm, cpu_attention.flash_attn_with_kvcache(q, kc, vc, cache_seqlens=before, page_table=bt, **extra)))
    width_used = sum(-(-n // 16) for n in lens)
    return fns, out, None, decode_bytes(lens, h, d, 2 if dtype == torch.bfloat16 else 4, append, width_used)


def best(timing, prefix):
    arms = [n for n in timing if n.split(" ")[0] == prefix]
    return min(arms, key=lambda n: timing[n]["gpu"]["median"]) if arms else None


def reference_rows(args, dev, flush, emit):
    for kind, specs in (("flash", FLASH), ("paged", PAGED)):
        for spec in specs:
            for dt in DT:
                name = label(kind, spec)
                if args.only not in name or args.dtype not in ("both", dt):
                    continue
                if PROFILE and (name, dt) != (PROFILE["row"], PROFILE["dtype"]):
                    continue
                torch.manual_seed(0)
                if kind == "flash":
                    fns, out, ref, work = flash_row(spec, DT[dt], dev)
                else:
                    fns, out, ref, work = paged_row(spec, DT[dt], dev)
                timing = measure(fns, flush, (name, dt))
                ours = best(timing, "ours")
                base = ref if ref in timing else None
                emit(kind, name, dt, spec, timing, ours, base, out, work)


def baseline_rows(args, dev, flush, emit):
    """The five BASELINE configs, each as its own row (cfg5 as two: the store of
    the prompts, then one decode step of the 32-step loop)."""
    rng = np.random.default_rng(0)
    rows = []
    if args.dtype in ("both", "bf16"):
        rows.append(("flash", "cfg1 prefill", "bf16", (1, 128, 16, 64, True)))
        rows.append(("flash", "cfg4 prefill (fused qkv)", "bf16", (4, 4096, 32, 128, True)))
        rows.append(("flash", "cfg4 cross", "bf16", (8, 2048, 32, 32, False, 1)))
    for kind, name, dt, spec in rows:
        if args.only not in name:
            continue
        fns, out, ref, work = flash_row(spec, DT[dt], dev, qkv_fused="fused" in name)
        timing = measure(fns, flush, (name, dt))
        if timing is not None:
            emit(kind, name, dt, spec, timing, "ours", ref if ref in timing else None, out, work)
    # cfg2: decode fp32 N=8 H=16 E=64 P=16, lens U[17,2047], append one token
    if args.dtype in ("both", "fp32") and args.only in "cfg2 decode":
        lens = [int(x) for x in rng.integers(17, 2048, size=8)]
        spec = (8, lens, 16, 64, True)
        fns, out, _, work = paged_row(spec, torch.float32, dev)
        fns = {k: f for k, f in fns.items() if k.endswith("p16")}
        timing = measure(fns, flush, ("cfg2 decode", "fp32"))
        if timing is not None:
            emit("paged", "cfg2 decode", "fp32", spec, timing, "ours p16", None, out, work)
    # cfg3: decode bf16 N=64 H=32 E=128 P=32, lens U[17,2047], random-permutation table, no append
    if args.dtype in ("both", "bf16") and args.only in "cfg3 decode":
        n, h, e, page = 64, 32, 128, 32
        lens = rng.integers(17, 2048, size=n)
        width = -(-2047 // page)
        g = torch.Generator(device=dev).manual_seed(0)
        table = torch.randperm(n * width, generator=g, device=dev).to(torch.int32).view(n, width)
        kc = torch.randn(n * width, h, page, e, generator=g, device=dev).to(torch.bfloat16)
        vc = torch.randn(n * width, h, page, e, generator=g, device=dev).to(torch.bfloat16)
        q = torch.randn(n, 1, h, e, generator=g, device=dev).to(torch.bfloat16)
        sl = torch.tensor(lens, dtype=torch.int32, device=dev)
        out = {}
        fns = {"ours p32": lambda: out.__setitem__("ours p32", cpu_attention.flash_attn_with_kvcache(
            q, kc, vc, cache_seqlens=sl, page_table=table))}
        work = decode_bytes([int(x) for x in lens], h, e, 2, False, sum(-(-int(x) // page) for x in lens))
        timing = measure(fns, flush, ("cfg3 decode", "bf16"))
        if timing is not None:
            emit("paged", "cfg3 decode", "bf16", (n, [int(x) for x in lens], h, e, False), timing,
                 "ours p32", None, out, work)
        del kc, vc
    # cfg5: store 128 prompts (U[64,1024], 10% padding slots) then decode steps with append
    if args.dtype in ("both", "bf16") and args.only in "cfg5 store + decode":
        n, h, e, page = 128, 32, 128, 16
        lens = rng.integers(64, 1025, size=n)
        total = int(lens.sum())
        steps = 32
        width = -(-(int(lens.max()) + steps) // page)
        nb = n * width
        g = torch.Generator(device=dev).manual_seed(5)
        table = torch.randperm(nb, generator=g, device=dev).to(torch.int32).view(n, width)
        kc = torch.zeros(nb, h, page, e, dtype=torch.bfloat16, device=dev)
        vc = torch.zeros_like(kc)
        tab = table.cpu().numpy()
        slots = np.concatenate([tab[i, np.arange(m) // page].astype(np.int64) * page + np.arange(m) % page
                                for i, m in enumerate(lens)])
        npad = len(slots) // 9  # about 10% of the entries are padding (-1)
        pad = np.zeros(len(slots) + npad, bool)
        pad[rng.choice(len(pad), npad, replace=False)] = True
        slot_map = np.full(len(pad), -1, np.int64)
        slot_map[~pad] = slots
        keep = slot_map >= 0
        key = torch.randn(len(slot_map), h, e, generator=g, device=dev).to(torch.bfloat16)
        val = torch.randn(len(slot_map), h, e, generator=g, device=dev).to(torch.bfloat16)
        sm = torch.from_numpy(slot_map).to(dev)
        fns = {"ours": lambda: cpu_attention.reshape_and_cache(key, val, kc, vc, sm)}
        stored = int(keep.sum())
        work = 2 * 2 * stored * h * e * 2 + len(slot_map) * 8
        timing = measure(fns, flush, ("cfg5 store", "bf16"))
        if timing is not None:
            emit("store", "cfg5 store", "bf16", (n, total, h, e, page), timing, "ours", None, {}, work)
        sl = torch.tensor(lens, dtype=torch.int32, device=dev)
        q = torch.randn(n, 1, h, e, generator=g, device=dev).to(torch.bfloat16)
        kn, vn = (torch.randn(n, 1, h, e, generator=g, device=dev).to(torch.bfloat16) for _ in range(2))
        out = {}
        step = [0]

        def decode_step():  # appends at lens + step (the loop's k-th step), attends lens + step + 1
            out["ours"] = cpu_attention.flash_attn_with_kvcache(q, kc, vc, k=kn, v=vn, cache_seqlens=sl + step[0],
                                                                page_table=table)
            step[0] = (step[0] + 1) % steps
        work = decode_bytes([int(m) + steps // 2 for m in lens], h, e, 2, True,
                            sum(-(-(int(m) + steps // 2) // page) for m in lens))
        timing = measure({"ours": decode_step}, flush, ("cfg5 decode step", "bf16"))
        if timing is not None:
            emit("paged", "cfg5 decode step", "bf16", (n, [int(x) for x in lens], h, e, True), timing,
                 "ours", None, out, work)


def row_work(kind, work):
    """A row's algorithmic bytes (prefill: q, k, v and out once)."""
    return work[1] if kind == "flash" else work


def main():
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--json", default="")
    ap.add_argument("--table", choices=("reference", "baseline", "both"), default="both")
    ap.add_argument("--only", default="", help="substring filter on row labels, e.g. 'N=8 '")
    ap.add_argument("--dtype", choices=("bf16", "fp32", "both"), default="both")
    ap.add_argument("--host-checks", choices=("on", "off"), default="on")
    ap.add_argument("--git", default="", help="commit label for the report (default: git rev-parse)")
    ap.add_argument("--counters", action="store_true",
                    help="add rocprofv3 columns (kernel time, HBM bytes, MFMA busy) to every row")
    ap.add_argument("--profile-row", nargs=3, metavar=("NAME", "DTYPE", "ARM"),
                    help="(used by --counters) run only this row's arm, for a rocprofv3 child")
    args = ap.parse_args()
    _kernel.set_host_checks(args.host_checks == "on")
    if not torch.cuda.is_available():
        print("bench: no GPU visible", file=sys.stderr)
        return 1
    if args.profile_row:
        PROFILE.update(row=args.profile_row[0], dtype=args.profile_row[1], arm=args.profile_row[2])
        # build only the profiled row (cfg5's two rows share one setup)
        args.only = "cfg5" if args.profile_row[0].startswith("cfg5") else args.profile_row[0]
        try:
            if args.table in ("reference", "both"):
                reference_rows(args, torch.device("cuda:0"), lambda: None, None)
            if args.table in ("baseline", "both"):
                baseline_rows(args, torch.device("cuda:0"), lambda: None, None)
        except Profiled:
            print("profiled", flush=True)
            return 0
        print(f"bench: no row {args.profile_row[0]!r} ({args.profile_row[1]})", file=sys.stderr)
        return 2
    dev = torch.device("cuda:0")
    flush = Flusher(dev)
    env = dict(machine=platform.node(), gpu=torch.cuda.get_device_name(0), host_checks=args.host_checks,
               git=args.git or sh("git", "-C", os.path.dirname(os.path.dirname(HERE)), "rev-parse", "--short", "HEAD"),
               torch=torch.__version__, hip=torch.version.hip, library=_kernel.module().version(),
               host_cores=_kernel.physical_cores())
    print(json.dumps(env), flush=True)
    rows = []

    def emit(kind, name, dt, spec, timing, ours, base, out, work):
        t = timing[ours]
        row = dict(kind=kind, name=name, dtype=dt, shape=spec, timing=timing, ours=ours, ref=base)
        sec = t["gpu"]["median"] * 1e-6
        if kind == "flash":
            row["tflops"] = work[0] / sec / 1e12
            row["gbs"] = work[1] / sec / 1e9
            row["roofline"] = dict(bound="mfma", peak=MFMA_TFLOPS[dt], frac=row["tflops"] / MFMA_TFLOPS[dt])
            rate = f"{row['tflops']:8.1f} TFLOP/s ({row['roofline']['frac']:.1%} of MFMA), {row['gbs']:6.0f} GB/s"
        else:
            row["gbs"] = work / sec / 1e9
            row["roofline"] = dict(bound="hbm", peak=HBM_GBS, frac=row["gbs"] / HBM_GBS)
            rate = f"{row['gbs']:8.0f} GB/s ({row['roofline']['frac']:.1%} of HBM)"
        line = (f"{kind:5s} {name:34s} {dt}  api {t['api']['median']:9.1f} us  gpu {t['gpu']['median']:9.1f} us"
                f"  {rate}  [{ours}]")
        if base:
            row["ratio"] = t["gpu"]["median"] / timing[base]["gpu"]["median"]
            row["max_diff"] = (out[ours].float() - out[base].float()).abs().max().item()
            line += f"  {base} gpu {timing[base]['gpu']['median']:9.1f} us  ratio {row['ratio']:.2f}" \
                    f"  diff {row['max_diff']:.1e}"
        if args.counters:
            import counters
            row["counters"] = counters.collect(
                name, dt, ours, kind, table="baseline" if name.startswith("cfg") else "reference",
                host_checks=args.host_checks)
            c = row["counters"]
            if c.get("kernel_us"):
                line += f"  | rocprof {c['kernel_us']:.1f} us"
            if c.get("hbm_bytes"):
                line += f", HBM {c['hbm_bytes'] / 1e6:.1f} MB ({c['hbm_bytes'] / max(row_work(kind, work), 1):.2f}x)"
            if c.get("mfma_util_pct") is not None:
                line += f", MFMA busy {c['mfma_util_pct']:.1f}%"
        print(line, flush=True)
        rows.append(row)
        if args.json:
            with open(args.json, "w") as f:
                json.dump(dict(environment=env, rows=rows), f)

    if args.table in ("reference", "both"):
        reference_rows(args, dev, flush, emit)
    if args.table in ("baseline", "both"):
        baseline_rows(args, dev, flush, emit)
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
