"""Benchmark of cpu-attention's hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--no-prefill]
                    [--no-configs] [--profile-pass] [--profile-configs] [--clock-trace N]

The headline step is one call of the paged decode over BASELINE cfg3 (bf16,
N=64 H=32 E=128 page 32, cache_seqlens U[17,2047], random-permutation page table,
no append): the north-star decode workload, HBM-bound.  ``value`` is the
whole-job throughput in algorithmic HBM bytes per second over the K timed steps
(inputs already resident in HBM), timed between two device synchronisations;
HIP events on the stream the kernels are launched on (torch's current stream)
bracket the timed region, split into TIMED_CHUNKS runs of consecutive steps, and
give ``us_per_call`` (the region's event time over K) and the roofline;
``us_per_call_median`` is the median of the runs' means.  No event sits between
the calls of a run: an event pair around every call adds ~2 us of GPU time of
its own.

Clock.  The chip needs tens of milliseconds of continuous work to settle at its
operating clock (the per-call trace from a cold start, ``--clock-trace``, shows
the climb).  Each leg therefore first runs its own workload back to back for a
fixed wall time (``clock_ramp_ms``, untimed, the call count reported), then the
W warm-up calls, then the K timed calls.  The timed window is thus the steady
state whatever W the caller passes.

The JSON line also carries:

* ``roofline`` for the decode kernel: algorithmic bytes per call / the event-timed
  average call duration against MI355X's 8 TB/s (``frac_cold`` and
  ``us_per_call_cold``: the same with the caches flushed before each call);
* ``prefill``: BASELINE cfg4 (bf16 causal N=4 L=S=4096 H=32 E=128, q/k/v
  strided chunks of a fused projection) in TFLOP/s against the 2.5 PFLOP/s dense
  bf16 MFMA peak, with its own roofline object;
* ``configs``: every other BASELINE config -- cfg1 (prefill N=1 L=S=128), cfg2
  (fp32 decode with a one-token append), cfg4's cross shape, and cfg5 (the 77k-slot
  reshape_and_cache staging and the 32 append+decode steps) -- each with its
  algorithmic bytes or FLOP, the roofline fraction, the event-timed device time
  warm (back to back) and cold (1 GiB written between calls, so neither L2 nor the
  256 MB MALL holds the inputs: the reference's method, benchmarks/bench.py:112-127),
  and the host wall time per call at the Python API;
* ``cpu_baseline``: the oracle's C port of the reference's CPU decode (the Mojo
  reference cannot be built here) on the box's physical host cores, over the whole
  cfg3 batch for CPU_BUDGET_S seconds (and the prefill port on one (batch, head) of
  cfg4 for as long), labelled as a substitute, with the reference's own published
  CPU figures beside it and, for the prefill, torch's CPU SDPA on the same cores
  (``prefill.cpu_baseline.torch_sdpa``) as a second substitute.

``roofline.traffic`` is the HBM bytes one call moves, from rocprofv3 --pmc runs of
``python bench.py --profile-pass`` (one 1 GiB device copy, then a few calls of
each workload): FETCH_SIZE and WRITE_SIZE per dispatch, each scaled by what the
same counter reads for the copy (TRAFFIC below; rerun the passes after a kernel
change).

Algorithmic bytes (decode) = sum over rows of 2*len*H*E*esize (K and V once) + q
+ out + page-table entries read + lengths (+ the appended token's read and write);
split-K partials are implementation traffic and are not counted.  Prefill FLOP =
4*E per visible (query, key) pair.
"""

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (ROOT, os.path.join(ROOT, "cpu-attention_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

import numpy as np  # noqa: E402
import torch  # noqa: E402

HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0
COPY_BYTES = 1 << 30  # the calibration copy of --profile-pass
FLUSH_BYTES = 1 << 30  # written between cold samples: > 2 x (256 MB MALL + L2)
RAMP_S = 0.2  # seconds of back-to-back calls before each leg's warm-up
TIMED_CHUNKS = 10  # event-timed runs the timed calls are split into
CPU_BUDGET_S = 8.0  # seconds of back-to-back calls per CPU baseline
METRIC = "decode HBM GB/s + µs/call; prefill TFLOP/s (bf16) vs MI355X roofline"

# rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE (KiB per dispatch) of --profile-pass on
# MI355X: the fifth of five calls of each workload (a decode call is its decode
# and combine dispatches), and what the same counter read for the run's 1 GiB
# calibration copy.
TRAFFIC = {
    "decode": {"fetch_kib": 543080.5 + 1310.5, "write_kib": 2630.3 + 400.0,
               "copy_fetch_kib": 524307.9, "copy_write_kib": 1048576.0},
    "prefill": {"fetch_kib": 294720.0, "write_kib": 132097.8,
                "copy_fetch_kib": 524315.2, "copy_write_kib": 1048576.0},
}

# The reference's published CPU figures (medians at its Python API, L2/L3 flushed,
# threads = physical cores; /root/reference/README.md:101-184,
# benchmarks/BENCHMARK.md:290-327).  c4d-standard-16 is an AMD EPYC 9B45 run with 8
# threads, the closest published host to an MI355X box.
PUBLISHED = {
    "decode": [{
        "workload": "paged decode bf16 N=32 L=1 S=1024 H=32 E=128 with a one-token append "
                    "(closest published row to cfg3)",
        "us_per_call": 9766, "GB/s": round(2 * 32 * 1025 * 32 * 128 * 2 / 9766e-6 / 1e9, 1),
        "host": "c4d-standard-16, AMD EPYC 9B45, 8 threads", "source": "README.md:156, BENCHMARK.md:327"}],
    "prefill": [{
        "workload": "flash_attn_func bf16 causal N=1 L=S=4096 H=32 E=128 (cfg4 at N=1)",
        "us_per_call": 56447, "TFLOP/s": round(4 * 32 * 128 * 4096 * 4097 / 2 / 56447e-6 / 1e12, 3),
        "host": "c4d-standard-16, AMD EPYC 9B45, 8 threads", "source": "README.md:127, BENCHMARK.md:300"}],
    "cfg1": [{"workload": "cfg1 exactly", "us_per_call": 56.5, "host": "c4d-standard-16 (8 threads)",
              "source": "README.md:124, BENCHMARK.md:294"}],
    "cfg2": [{"workload": "decode fp32 N=8 H=16 E=64 lens [17,255,1023,1025,33,513,2047,64] + append "
                          "(closest published row to cfg2)", "us_per_call": 803,
              "host": "c4d-standard-16 (8 threads)", "source": "README.md:167, BENCHMARK.md:322"}],
}


def traffic_bytes(name):
    """HBM bytes of one call: each counter scaled by its reading for a known copy."""
    if name not in TRAFFIC:
        return None
    t = TRAFFIC[name]
    return int(t["fetch_kib"] * COPY_BYTES / t["copy_fetch_kib"] + t["write_kib"] * COPY_BYTES / t["copy_write_kib"])


# ---------------------------------------------------------------------------
# timing
# ---------------------------------------------------------------------------
def ramp(fn, seconds=RAMP_S):
    """Runs fn back to back for `seconds` of wall time (the clock settles); returns
    the number of calls."""
    torch.cuda.synchronize()
    n, t0 = 0, time.perf_counter()
    while True:
        for _ in range(8):
            fn()
        n += 8
        torch.cuda.synchronize()
        if time.perf_counter() - t0 >= seconds:
            return n


def timed(fn, steps, warmup, ramp_s=RAMP_S, chunks=TIMED_CHUNKS):
    """Clock ramp, `warmup` untimed calls, then `steps` back-to-back calls between
    two device synchronisations.  Events on the current stream split the timed
    calls into `chunks` runs of consecutive calls (no event between the calls of
    a run: an event pair around every call adds its own ~2 us of GPU time, which
    is a tenth of a small call).  Returns (wall seconds over the timed calls, the
    event milliseconds per call of each run, ramp calls); the mean call is the
    event time of the whole region over `steps`."""
    nramp = ramp(fn, ramp_s) if ramp_s > 0 else 0
    for _ in range(warmup):
        fn()
    n = max(1, min(chunks, steps))
    sizes = [steps // n + (1 if i < steps % n else 0) for i in range(n)]
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(n + 1)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    ev[0].record()
    for i, size in enumerate(sizes):
        for _ in range(size):
            fn()
        ev[i + 1].record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    return wall, [ev[i].elapsed_time(ev[i + 1]) / size for i, size in enumerate(sizes)], nramp


def region_ms(ms, steps):
    """Mean event milliseconds per call over the whole timed region (runs weighted
    by their call counts)."""
    n = len(ms)
    sizes = [steps // n + (1 if i < steps % n else 0) for i in range(n)]
    return sum(m * s for m, s in zip(ms, sizes)) / steps


class Flush:
    """1 GiB written before each cold sample, so no cache holds the inputs."""

    def __init__(self, dev):
        self.buf = torch.empty(FLUSH_BYTES // 4, dtype=torch.float32, device=dev)

    def __call__(self):
        self.buf.fill_(1.0)


def cold(fn, flush, samples=15, warmup=3):
    """Median (and min/max) event time of fn with the caches flushed before each
    call (3 untimed calls first), as the reference's benchmark does."""
    for _ in range(warmup):
        flush()
        fn()
    ms = []
    for _ in range(samples):
        flush()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        fn()
        b.record()
        torch.cuda.synchronize()
        ms.append(a.elapsed_time(b))
    return float(np.median(ms)), float(np.min(ms)), float(np.max(ms))


def api_wall(fn, calls=200):
    """Host wall time per call at the Python API over back-to-back calls (one
    synchronisation at the end), in microseconds."""
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(calls):
        fn()
    torch.cuda.synchronize()
    return (time.perf_counter() - t0) / calls * 1e6


def measure(fn, flush, work, unit, steps=100, warmup=10, cold_samples=15, peak=None, api_calls=200):
    """One config entry: warm and cold device time, API wall time, and the rate
    of `work` (bytes or FLOP per call) against `peak`."""
    _, ms, nramp = timed(fn, steps, warmup, ramp_s=0.05)
    warm = region_ms(ms, steps)
    cmed, cmin, cmax = cold(fn, flush, cold_samples)
    scale = 1e9 if unit == "GB/s" else 1e12
    rate = work / (warm * 1e-3) / scale
    rate_cold = work / (cmed * 1e-3) / scale
    out = {"us_per_call": round(warm * 1e3, 2), "us_per_call_median": round(float(np.median(ms)) * 1e3, 2),
           "us_per_call_cold": round(cmed * 1e3, 2), "us_per_call_cold_min_max": [round(cmin * 1e3, 2),
                                                                                  round(cmax * 1e3, 2)],
           "api_us_per_call": round(api_wall(fn, api_calls), 2), "value": round(rate, 2),
           "value_cold": round(rate_cold, 2), "unit": unit, "clock_ramp_calls": nramp,
           "steps": steps, "warmup": warmup, "cold_samples": cold_samples}
    if peak:
        out["roofline"] = {"bound": "hbm" if unit == "GB/s" else "mfma", "achieved": round(rate, 1),
                           "peak": peak, "unit": unit, "frac": round(rate / peak, 4),
                           "frac_cold": round(rate_cold / peak, 4)}
    return out


# ---------------------------------------------------------------------------
# workloads (seeded synthetic inputs of the BASELINE shapes)
# ---------------------------------------------------------------------------
def decode_bytes(lens, h, e, esize, page, append):
    """Algorithmic bytes of one decode call: K and V of every attended key once,
    q and out, the page-table entries and lengths read, and with an append the new
    token's read (k/v inputs) and write (cache)."""
    att = [int(m) + (1 if append else 0) for m in lens]
    n = len(lens)
    kv = sum(2 * a * h * e * esize for a in att)
    io = 2 * n * h * e * esize + sum(-(-a // page) for a in att) * 4 + n * 4
    new = 4 * n * h * e * esize if append else 0
    return kv + io + new


def decode_workload(dev, seed=0):
    """cfg3: bf16 N=64 H=32 E=128 page 32, lens U[17,2047], random-permutation page table."""
    n, h, e, page = 64, 32, 128, 32
    rng = np.random.default_rng(seed)
    lens = rng.integers(17, 2048, size=n)
    width = -(-2047 // page)
    nb = n * width
    g = torch.Generator(device=dev).manual_seed(seed)
    table = torch.randperm(nb, generator=g, device=dev).to(torch.int32).view(n, width)
    kc = torch.randn(nb, h, page, e, generator=g, device=dev).to(torch.bfloat16)
    vc = torch.randn(nb, h, page, e, generator=g, device=dev).to(torch.bfloat16)
    q = torch.randn(n, 1, h, e, generator=g, device=dev).to(torch.bfloat16)
    seqlens = torch.tensor(lens, dtype=torch.int32, device=dev)
    return dict(n=n, h=h, e=e, page=page, lens=lens, table=table, kc=kc, vc=vc, q=q,
                seqlens=seqlens, bytes=decode_bytes(lens, h, e, 2, page, False))


def prefill_workload(dev):
    """cfg4: q/k/v [4, 4096, 32, 128] bf16 as strided chunks of one fused projection."""
    N, L, H, E = 4, 4096, 32, 128
    g = torch.Generator(device=dev).manual_seed(1)
    qkv = torch.randn(N * L, 3 * H * E, generator=g, device=dev).to(torch.bfloat16)
    q, k, v = (qkv[:, i * H * E:(i + 1) * H * E].view(N, L, H, E) for i in range(3))
    return qkv, q, k, v


def causal_flop(n, h, e, sq, sk):
    """4*E per visible (query, key) pair, bottom-right causal."""
    diag = sk - sq
    vis = sum(max(0, min(sk, i + diag + 1)) for i in range(sq))
    return 4 * n * h * e * vis


def paged_caches(dev, lens_cap, h, e, page, dtype, seed):
    """A random-permutation page table with room for `lens_cap[i]` keys per
    sequence, and caches of exactly that many blocks (NaN-free zeros)."""
    g = torch.Generator(device=dev).manual_seed(seed)
    pages = [-(-int(c) // page) for c in lens_cap]
    width, nb = max(pages), sum(pages)
    perm = torch.randperm(nb, generator=g, device=dev).to(torch.int32)
    table = torch.zeros(len(pages), width, dtype=torch.int32, device=dev)
    start = 0
    for i, p in enumerate(pages):
        table[i, :p] = perm[start:start + p]
        start += p
    kc = torch.zeros(nb, h, page, e, dtype=dtype, device=dev)
    vc = torch.zeros_like(kc)
    return table, kc, vc


def slots_for(table, lens, page, pad_frac, rng):
    """Slot mapping of every prompt token (position j of sequence i at
    table[i, j // page] * page + j % page), with about `pad_frac` of -1 padding
    entries interleaved at random positions."""
    t = table.cpu().numpy().astype(np.int64)
    real = np.concatenate([t[i, np.arange(m) // page] * page + np.arange(m) % page
                           for i, m in enumerate(lens)])
    npad = int(round(len(real) * pad_frac / (1 - pad_frac)))
    out = np.full(len(real) + npad, -1, np.int64)
    keep = np.sort(rng.choice(len(out), size=len(real), replace=False))
    out[keep] = real
    return out, len(real)


def run_configs(dev, mod, rt, profile_calls=0):
    """The BASELINE configs other than the headline decode and prefill.  With
    ``profile_calls``, nothing is timed: each config's call runs that many times
    (cfg5's 32-step loop once), for a counter run to read."""
    from cpu_attention import flash_attn_func, flash_attn_with_kvcache, reshape_and_cache

    flush = Flush(dev)
    res = {}

    def measure_or_run(fn, *args, **kw):
        if not profile_calls:
            return measure(fn, *args, **kw)
        for _ in range(profile_calls):
            fn()
        torch.cuda.synchronize()
        return {}

    # cfg1: prefill bf16 N=1 L=S=128 H=16 E=64 causal (latency-bound: 34 MFLOP).
    g = torch.Generator(device=dev).manual_seed(2)
    q, k, v = (torch.randn(1, 128, 16, 64, generator=g, device=dev).to(torch.bfloat16) for _ in range(3))
    flop = causal_flop(1, 16, 64, 128, 128)
    res["cfg1"] = {"workload": "flash_attn_func bf16 causal N=1 L=S=128 H=16 E=64", "algorithmic_flop": flop,
                   **measure_or_run(lambda: flash_attn_func(q, k, v, causal=True), flush, flop, "TFLOP/s",
                             peak=BF16_PEAK_TFLOPS),
                   "published_cpu": PUBLISHED["cfg1"]}
    del q, k, v

    # cfg2: decode fp32 N=8 H=16 E=64 page 16, lens U[17,2047], caches filled by
    # reshape_and_cache, a one-token append each call (at the same position).
    n, h, e, page = 8, 16, 64, 16
    rng = np.random.default_rng(3)
    lens = rng.integers(17, 2048, size=n)
    table, kc, vc = paged_caches(dev, lens + 1, h, e, page, torch.float32, seed=3)
    slots, _ = slots_for(table, lens, page, 0.0, rng)
    gk = torch.Generator(device=dev).manual_seed(3)
    kv = torch.randn(2, len(slots), h, e, generator=gk, device=dev)
    reshape_and_cache(kv[0], kv[1], kc, vc, torch.from_numpy(slots).to(dev))
    q, kn, vn = (torch.randn(n, 1, h, e, generator=gk, device=dev) for _ in range(3))
    seqlens = torch.tensor(lens, dtype=torch.int32, device=dev)
    nbytes = decode_bytes(lens, h, e, 4, page, True)
    res["cfg2"] = {"workload": "flash_attn_with_kvcache fp32 N=8 H=16 E=64 page 16, lens U[17,2047], "
                               "random-permutation page table, caches filled by reshape_and_cache, "
                               "one-token append per call",
                   "algorithmic_bytes": nbytes,
                   **measure_or_run(lambda: flash_attn_with_kvcache(q, kc, vc, k=kn, v=vn, cache_seqlens=seqlens,
                                                             page_table=table), flush, nbytes, "GB/s",
                             peak=HBM_PEAK_GBS),
                   "published_cpu": PUBLISHED["cfg2"]}
    del kc, vc, kv

    # cfg4 cross: N=8 L=1 S=2048 H=32 E=32, non-causal bf16 (HBM-bound).
    g = torch.Generator(device=dev).manual_seed(4)
    q = torch.randn(8, 1, 32, 32, generator=g, device=dev).to(torch.bfloat16)
    k, v = (torch.randn(8, 2048, 32, 32, generator=g, device=dev).to(torch.bfloat16) for _ in range(2))
    nbytes = 2 * q.numel() * 2 + 2 * k.numel() * 2
    res["cfg4_cross"] = {"workload": "flash_attn_func bf16 non-causal N=8 L=1 S=2048 H=32 E=32",
                         "algorithmic_bytes": nbytes,
                         **measure_or_run(lambda: flash_attn_func(q, k, v, causal=False), flush, nbytes, "GB/s",
                                   peak=HBM_PEAK_GBS)}
    del q, k, v

    # cfg5: N=128 H=32 E=128 page 16 bf16; 128 prompts of U[64,1024] tokens staged by
    # one reshape_and_cache (10% of the slot entries -1), then 32 steps that each
    # append one token per sequence and attend.
    n, h, e, page, nsteps = 128, 32, 128, 16, 32
    rng = np.random.default_rng(5)
    lens = rng.integers(64, 1025, size=n)
    table, kc, vc = paged_caches(dev, lens + nsteps, h, e, page, torch.bfloat16, seed=5)
    slots, nreal = slots_for(table, lens, page, 0.10, rng)
    g = torch.Generator(device=dev).manual_seed(5)
    key = torch.randn(len(slots), h, e, generator=g, device=dev).to(torch.bfloat16)
    val = torch.randn(len(slots), h, e, generator=g, device=dev).to(torch.bfloat16)
    sl = torch.from_numpy(slots).to(dev)
    store_bytes = 4 * nreal * h * e * 2 + 8 * len(slots)
    res["cfg5_store"] = {"workload": f"reshape_and_cache bf16 H=32 E=128 page 16: {len(slots)} slot entries "
                                     f"({len(slots) - nreal} of them -1) for 128 prompts of U[64,1024] tokens",
                         "algorithmic_bytes": store_bytes,
                         **measure_or_run(lambda: reshape_and_cache(key, val, kc, vc, sl), flush, store_bytes, "GB/s",
                                   steps=30, warmup=3, cold_samples=10, peak=HBM_PEAK_GBS, api_calls=20)}
    del key, val
    qs = torch.randn(nsteps, n, 1, h, e, generator=g, device=dev).to(torch.bfloat16)
    ks = torch.randn(nsteps, n, 1, h, e, generator=g, device=dev).to(torch.bfloat16)
    vs = torch.randn(nsteps, n, 1, h, e, generator=g, device=dev).to(torch.bfloat16)
    lens_t = [torch.tensor(lens + s, dtype=torch.int32, device=dev) for s in range(nsteps)]
    step_bytes = [decode_bytes(lens + s, h, e, 2, page, True) for s in range(nsteps)]

    def loop():
        for s in range(nsteps):
            flash_attn_with_kvcache(qs[s], kc, vc, k=ks[s], v=vs[s], cache_seqlens=lens_t[s], page_table=table)

    if profile_calls:
        loop()
        torch.cuda.synchronize()
        return res
    nramp = ramp(loop, 0.05)
    loop()
    # The rate: the 32 steps back to back between two events, three times.
    reps, total_ms = 3, 0.0
    for _ in range(reps):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        a.record()
        loop()
        b.record()
        torch.cuda.synchronize()
        total_ms += a.elapsed_time(b) / reps
    # The spread over the steps: one more pass with an event pair around each step.
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(nsteps)]
    torch.cuda.synchronize()
    for s, (a, b) in enumerate(ev):
        a.record()
        flash_attn_with_kvcache(qs[s], kc, vc, k=ks[s], v=vs[s], cache_seqlens=lens_t[s], page_table=table)
        b.record()
    torch.cuda.synchronize()
    per_step = np.array([a.elapsed_time(b) for a, b in ev])
    rate = sum(step_bytes) / (total_ms * 1e-3) / 1e9
    # cold: the caches flushed before every step (the K/V of the other layers of a
    # real model would pass through them between two steps of this one)
    cold_ms = np.zeros(nsteps)
    for s, (a, b) in enumerate(ev):
        flush()
        a.record()
        flash_attn_with_kvcache(qs[s], kc, vc, k=ks[s], v=vs[s], cache_seqlens=lens_t[s], page_table=table)
        b.record()
    torch.cuda.synchronize()
    cold_ms += [a.elapsed_time(b) for a, b in ev]
    cold_rate = sum(step_bytes) / (float(cold_ms.sum()) * 1e-3) / 1e9
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    loop()
    torch.cuda.synchronize()
    api = (time.perf_counter() - t0) / nsteps * 1e6
    res["cfg5_step"] = {"workload": "32 steps of flash_attn_with_kvcache bf16 N=128 H=32 E=128 page 16, each "
                                    "appending one token per sequence and attending (lens U[64,1024] + step)",
                        "algorithmic_bytes_per_step": int(np.mean(step_bytes)),
                        "us_per_step": round(total_ms / nsteps * 1e3, 2),
                        "us_per_step_min_max": [round(float(per_step.min()) * 1e3, 2),
                                                round(float(per_step.max()) * 1e3, 2)],
                        "us_per_step_cold": round(float(cold_ms.mean()) * 1e3, 2),
                        "api_us_per_step": round(api, 2), "value": round(rate, 2),
                        "value_cold": round(cold_rate, 2), "unit": "GB/s",
                        "clock_ramp_calls": nramp * nsteps, "repeats": reps,
                        "roofline": {"bound": "hbm", "achieved": round(rate, 1), "peak": HBM_PEAK_GBS,
                                     "unit": "GB/s", "frac": round(rate / HBM_PEAK_GBS, 4),
                                     "frac_cold": round(cold_rate / HBM_PEAK_GBS, 4)}}
    return res


# ---------------------------------------------------------------------------
# CPU baseline (the oracle's C port: test infrastructure, timed here only)
# ---------------------------------------------------------------------------
def host_cpu():
    """The host CPU's model name and whether it has AVX-512 (the C port's wide
    tiles), from /proc/cpuinfo."""
    model, flags = "unknown", ""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name") and model == "unknown":
                    model = line.split(":", 1)[1].strip()
                elif line.startswith("flags") and not flags:
                    flags = line
    except OSError:
        pass
    return f"{model}{', AVX-512' if ' avx512f' in flags else ''}"


def cpu_decode_baseline(w, budget_s=CPU_BUDGET_S):
    """The C port of the reference's CPU decode on the host's physical cores, over the
    whole cfg3 batch, called back to back for ``budget_s`` seconds."""
    from cpu_attention import _kernel as K
    from oracle import cport

    ns = w["n"]
    page, h, e = w["page"], w["h"], w["e"]
    lens = w["lens"][:ns]
    pages = [-(-int(m) // page) for m in lens]
    blocks = torch.cat([w["table"][i, :p].long() for i, p in enumerate(pages)])
    kc = w["kc"][blocks].view(torch.int16).cpu().numpy().view(np.uint16)
    vc = w["vc"][blocks].view(torch.int16).cpu().numpy().view(np.uint16)
    table = np.zeros((ns, max(pages)), np.int32)
    start = 0
    for i, p in enumerate(pages):
        table[i, :p] = np.arange(start, start + p)
        start += p
    q = w["q"][:ns, 0].contiguous().view(torch.int16).cpu().numpy().view(np.uint16)
    threads = K.physical_cores()
    cport.decode(q, kc, vc, lens, table, page, e ** -0.5, True, threads)  # warm
    reps, t0 = 0, time.perf_counter()
    while True:
        cport.decode(q, kc, vc, lens, table, page, e ** -0.5, True, threads)
        reps += 1
        if time.perf_counter() - t0 >= budget_s and reps >= 3:
            break
    dt = (time.perf_counter() - t0) / reps
    nbytes = sum(2 * int(m) * h * e * 2 for m in lens) + 2 * ns * h * e * 2
    return {"value": round(nbytes / dt / 1e9, 3), "unit": "GB/s", "cores": threads, "host": host_cpu(), "kind": "port",
            "substitute": True,
            "note": "the reference's Mojo CPU path cannot be built (mojo needs a network install); this is "
                    "the oracle's C/OpenMP port of its decode algorithm, a substitute, with the reference's "
                    "published CPU figures beside it",
            "sample": f"C port (oracle/ca_oracle.c, OpenMP) of the reference's paged decode on the "
                      f"whole cfg3 batch ({ns} sequences, {nbytes / 1e6:.0f} MB of K/V, bf16), "
                      f"{reps} calls in {reps * dt:.1f} s, {dt * 1e3:.2f} ms/call",
            "published": PUBLISHED["decode"]}


def cpu_prefill_baseline(budget_s=CPU_BUDGET_S):
    """The C port of the reference's prefill on the host's physical cores, one
    (batch, head) of cfg4 per call, called back to back for ``budget_s`` seconds."""
    from cpu_attention import _kernel as K
    from oracle import bf16, cport

    b, L, h, e = 1, 4096, 1, 128
    rng = np.random.default_rng(1)
    q, k, v = (bf16.from_float(rng.standard_normal((b, L, h, e)).astype(np.float32)) for _ in range(3))
    threads = K.physical_cores()
    reps, t0 = 0, time.perf_counter()
    while True:
        cport.flash(q, k, v, e ** -0.5, True, True, threads)
        reps += 1
        if time.perf_counter() - t0 >= budget_s and reps >= 3:
            break
    dt = (time.perf_counter() - t0) / reps
    flop = 4 * b * h * e * L * (L + 1) / 2
    rate = flop / dt / 1e12
    pub = PUBLISHED["prefill"][0]["TFLOP/s"]
    return {"value": round(rate, 4), "unit": "TFLOP/s", "cores": threads, "host": host_cpu(), "kind": "port",
            "substitute": True,
            "note": "the oracle's fp32 C port of the reference's prefill, AVX-512 or AVX2 register tiles "
                    f"(the Mojo path cannot be built here); its rate is {rate / pub:.2f}x the reference's "
                    "published one (8 EPYC 9B45 threads, bf16 dot products), which stays the figure to "
                    "compare with",
            "sample": f"C port of the reference's prefill, one (batch, head) of the config "
                      f"(L=S=4096 E=128 causal bf16), {reps} calls in {reps * dt:.1f} s, {dt * 1e3:.1f} ms/call",
            "published": PUBLISHED["prefill"], "torch_sdpa": cpu_sdpa_baseline(threads, budget_s / 2)}


def cpu_sdpa_baseline(threads, budget_s):
    """torch's CPU scaled_dot_product_attention on the same prefill shape (8 of its
    heads per call, bf16, causal), on the host's physical cores: a second
    substitute for the reference's CPU path, not the reference."""
    old = torch.get_num_threads()
    torch.set_num_threads(threads)
    try:
        h, L, e = 8, 4096, 128
        g = torch.Generator().manual_seed(2)
        q, k, v = (torch.randn(1, h, L, e, generator=g).bfloat16() for _ in range(3))
        sdpa = torch.nn.functional.scaled_dot_product_attention
        sdpa(q, k, v, is_causal=True)  # warm
        reps, t0 = 0, time.perf_counter()
        while True:
            sdpa(q, k, v, is_causal=True)
            reps += 1
            if time.perf_counter() - t0 >= budget_s and reps >= 3:
                break
        dt = (time.perf_counter() - t0) / reps
    finally:
        torch.set_num_threads(old)
    flop = 4 * h * e * L * (L + 1) / 2
    return {"value": round(flop / dt / 1e12, 4), "unit": "TFLOP/s", "cores": threads, "kind": "torch",
            "sample": f"torch {torch.__version__} CPU SDPA, bf16 causal [1, 8 heads, 4096, 128], {reps} calls "
                      f"in {reps * dt:.1f} s, {dt * 1e3:.1f} ms/call"}


# ---------------------------------------------------------------------------
# profile and trace passes
# ---------------------------------------------------------------------------
def profile_pass(dev, mod, rt, calls=5):
    """No timing: one 1 GiB device copy (the counters' calibration), then `calls`
    calls of the decode (cfg3) and of the prefill (cfg4); a counter summary
    takes the last call of each."""
    src = torch.ones(COPY_BYTES // 4, dtype=torch.float32, device=dev)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    dst.copy_(src)
    torch.cuda.synchronize()
    del src, dst
    w = decode_workload(dev)
    out = torch.empty_like(w["q"])
    for _ in range(calls):
        assert mod.decode(rt, w["q"], w["kc"], w["vc"], None, None, None, w["seqlens"], w["table"],
                          None, out) is not None
    torch.cuda.synchronize()
    del w, out
    torch.cuda.empty_cache()
    qkv, q, k, v = prefill_workload(dev)
    for _ in range(calls):
        r = mod.flash(rt, q, k, v, None, True, 0, 0)
        assert r is not None and not isinstance(r, int)
    torch.cuda.synchronize()
    print("profile pass done", flush=True)


def profile_configs(dev, mod, rt, calls=5):
    """No timing: one 1 GiB device copy (the counters' calibration), then `calls`
    calls of each other BASELINE config (cfg1, cfg2, cfg4's cross shape, cfg5's
    staging store) and one pass of cfg5's 32 append+decode steps."""
    src = torch.ones(COPY_BYTES // 4, dtype=torch.float32, device=dev)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    dst.copy_(src)
    torch.cuda.synchronize()
    del src, dst
    torch.cuda.empty_cache()
    run_configs(dev, mod, rt, profile_calls=calls)
    print("profile configs done", flush=True)


def clock_trace(dev, mod, rt, calls):
    """`calls` back-to-back prefill calls (cfg4) from a cold start, each bracketed by
    events: one line per call (index, µs), then a summary."""
    qkv, q, k, v = prefill_workload(dev)
    torch.cuda.synchronize()
    time.sleep(2.0)  # let the chip idle down first
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(calls)]
    for a, b in ev:
        a.record()
        r = mod.flash(rt, q, k, v, None, True, 0, 0)
        b.record()
    torch.cuda.synchronize()
    assert r is not None and not isinstance(r, int)
    us = [a.elapsed_time(b) * 1e3 for a, b in ev]
    t = np.cumsum(us) / 1e3
    for i, (x, tt) in enumerate(zip(us, t)):
        print(f"call {i:4d}  t={tt:8.2f} ms  {x:8.1f} us")
    for lo, hi in ((0, 10), (10, 50), (50, 100), (100, 200), (200, 400), (400, calls)):
        if hi <= calls and hi > lo:
            print(f"calls {lo}-{hi - 1}: mean {np.mean(us[lo:hi]):.1f} us")
    print(f"steady state (last half): mean {np.mean(us[calls // 2:]):.1f} us, "
          f"median {np.median(us[calls // 2:]):.1f} us", flush=True)


def progress(what, t0):
    """One line on stderr per finished leg (stdout carries only the JSON line)."""
    print(f"bench: {what} done ({time.perf_counter() - t0:.1f} s)", file=sys.stderr, flush=True)


def main():
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-prefill", action="store_true", help="skip the prefill line")
    ap.add_argument("--no-configs", action="store_true", help="skip the other BASELINE configs")
    ap.add_argument("--profile-pass", action="store_true",
                    help="no timing: one 1 GiB device copy, then a few decode and prefill calls "
                         "(for rocprofv3 --pmc runs)")
    ap.add_argument("--profile-configs", action="store_true",
                    help="no timing: one 1 GiB device copy, then a few calls of each other config "
                         "(for rocprofv3 --pmc runs)")
    ap.add_argument("--clock-trace", type=int, default=0, metavar="N",
                    help="print the event time of N back-to-back prefill calls from a cold start")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: the ops run within one device and this build "
              "has no multi-GPU path (sequences or heads would shard across GPUs with no "
              "cross-GPU traffic inside a call). Use --gpus 1.",
              file=sys.stderr)
        sys.exit(2)

    from cpu_attention import _kernel as K

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    mod, rt = K.module(), K.runtime()
    K.set_host_checks(False)  # no host reads inside the timed loops

    if args.profile_pass:
        profile_pass(dev, mod, rt)
        return
    if args.profile_configs:
        profile_configs(dev, mod, rt)
        return
    if args.clock_trace:
        clock_trace(dev, mod, rt, args.clock_trace)
        return

    t0 = time.perf_counter()
    w = decode_workload(dev)
    out = torch.empty_like(w["q"])

    def step():
        r = mod.decode(rt, w["q"], w["kc"], w["vc"], None, None, None, w["seqlens"], w["table"],
                       None, out)
        assert r is not None

    wall, ms, nramp = timed(step, args.steps, args.warmup)
    call_ms = region_ms(ms, args.steps)
    gbs_kernel = w["bytes"] / (call_ms * 1e-3) / 1e9
    # cold: caches flushed before each sample (the 1 GiB fill leaves the caches
    # full of dirty lines, whose write-back the call then pays for)
    flush = Flush(dev)
    cmed, cmin, cmax = cold(step, flush, 15)
    value = w["bytes"] * args.steps / wall / 1e9
    res = {
        "metric": METRIC, "value": round(value, 2), "unit": "GB/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(wall / args.steps * 1e3, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": "paged decode flash_attn_with_kvcache bf16 N=64 H=32 E=128 page=32 "
                               "cache_seqlens U[17,2047] random-permutation page_table, no append",
                   "global_batch": w["n"], "seq_len": "17..2047", "parallelism": "none (1 GPU)"},
        "clock_ramp_ms": RAMP_S * 1e3, "clock_ramp_calls": nramp,
        "us_per_call": round(call_ms * 1e3, 2),
        "us_per_call_median": round(float(np.median(ms)) * 1e3, 2),
        "us_per_call_cold": round(cmed * 1e3, 2), "us_per_call_cold_min_max": [round(cmin * 1e3, 2),
                                                                               round(cmax * 1e3, 2)],
        "roofline": {"bound": "hbm", "achieved": round(gbs_kernel, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(gbs_kernel / HBM_PEAK_GBS, 4),
                     "frac_cold": round(w["bytes"] / (cmed * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                     "traffic": traffic_bytes("decode"),
                     "kernel": "decode_tiles_kernel<128,bf16,64-key tiles> + decode_tiles_combine_kernel "
                               "(the call's two dispatches, timed together)",
                     "algorithmic_bytes": w["bytes"]},
    }
    del w
    torch.cuda.empty_cache()
    progress("decode (cfg3)", t0)

    if not args.no_prefill:
        N, L, H, E = 4, 4096, 32, 128
        qkv, q, k, v = prefill_workload(dev)

        def pstep():
            r = mod.flash(rt, q, k, v, None, True, 0, 0)
            assert r is not None and not isinstance(r, int)

        psteps, pwarm = max(20, args.steps // 2), args.warmup
        pwall, pms, pramp = timed(pstep, psteps, pwarm)
        flop = causal_flop(N, H, E, L, L)
        pcall = region_ms(pms, psteps)
        pcmed, pcmin, pcmax = cold(pstep, flush, 10)
        tf = flop / (pcall * 1e-3) / 1e12
        res["prefill"] = {
            "workload": "flash_attn_func bf16 causal N=4 L=S=4096 H=32 E=128, q/k/v strided "
                        "chunks of a fused [N*L, 3*H*E] projection",
            "value": round(flop * psteps / pwall / 1e12, 2), "unit": "TFLOP/s",
            "steps": psteps, "warmup": pwarm, "clock_ramp_ms": RAMP_S * 1e3, "clock_ramp_calls": pramp,
            "us_per_call": round(pcall * 1e3, 1), "us_per_call_median": round(float(np.median(pms)) * 1e3, 1),
            "us_per_call_cold": round(pcmed * 1e3, 1),
            "us_per_call_cold_min_max": [round(pcmin * 1e3, 1), round(pcmax * 1e3, 1)],
            "roofline": {"bound": "mfma", "achieved": round(tf, 1), "peak": BF16_PEAK_TFLOPS,
                         "unit": "TFLOP/s", "frac": round(tf / BF16_PEAK_TFLOPS, 4),
                         "frac_cold": round(flop / (pcmed * 1e-3) / 1e12 / BF16_PEAK_TFLOPS, 4),
                         "traffic": traffic_bytes("prefill"), "kernel": "flash_bf16_p64_kernel<128, false>",
                         "algorithmic_flop": flop},
        }
        del qkv, q, k, v
        torch.cuda.empty_cache()
        progress("prefill (cfg4)", t0)

    if not args.no_configs:
        res["configs"] = run_configs(dev, mod, rt)
        torch.cuda.empty_cache()
        progress("configs", t0)

    if not args.no_cpu:
        w = decode_workload(dev)
        res["cpu_baseline"] = cpu_decode_baseline(w)
        del w
        progress("CPU decode baseline", t0)
        if not args.no_prefill:
            res["prefill"]["cpu_baseline"] = cpu_prefill_baseline()
            progress("CPU prefill baseline", t0)
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
