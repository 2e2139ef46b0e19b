"""Benchmark of cpu-attention's hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--no-prefill]

A step is one call of the paged decode over BASELINE config 2 (bf16, N=64 H=32
E=128 page 32, cache_seqlens U[17,2047], random-permutation page table, no
append): the north-star decode workload, HBM-bound.  W untimed steps (by default
enough to carry the chip past its ~25 ms climb to the operating clock), then K
timed steps between two device synchronisations; every step is also bracketed by
HIP events on the stream the kernels are launched on (torch's current stream).
``value`` is the whole-job throughput in algorithmic HBM bytes per second over
the timed region (inputs already resident in HBM).  The JSON line also carries:

* ``roofline`` for the decode kernels: algorithmic bytes per call / the event-
  timed average call duration against MI355X's 8 TB/s;
* ``prefill``: BASELINE config 3 (bf16 causal N=4 L=S=4096 H=32 E=128, q/k/v
  strided chunks of a fused projection) in TFLOP/s against the 2.5 PFLOP/s
  dense bf16 MFMA peak, with its own roofline object;
* ``cpu_baseline``: the oracle's C port of the reference's CPU decode (the Mojo
  reference cannot be built here) on the box's host cores, on a bounded sample
  of the same workload.

``roofline.traffic`` is the HBM bytes one call moves, from rocprofv3 --pmc runs
of ``python bench.py --profile-pass`` (one 1 GiB device copy, then one call of
each workload): FETCH_SIZE and WRITE_SIZE per dispatch, each scaled by what the
same counter reads for the copy (TRAFFIC below; rerun the passes after a kernel
change).

Algorithmic bytes (decode) = sum over rows of 2*len*H*E*2 (K and V once) + q + out
+ page-table entries read + lengths; split-K partials are implementation traffic
and are not counted.  Prefill FLOP = 4*E per visible (query, key) pair.
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

# rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE (KiB per dispatch) of --profile-pass on
# MI355X: the calibration copy, then the decode kernels and the prefill kernel.
TRAFFIC = {
    "copy": {"fetch_kib": 524307.7, "write_kib": 1048576.0},
    "decode": {"fetch_kib": 543466.4, "write_kib": 512.0},
    "prefill": {"fetch_kib": 312573.0, "write_kib": 152576.0},
}


def traffic_bytes(name):
    """HBM bytes of one call: each counter scaled by its reading for a known copy."""
    t, c = TRAFFIC[name], TRAFFIC["copy"]
    return int(t["fetch_kib"] * COPY_BYTES / c["fetch_kib"] + t["write_kib"] * COPY_BYTES / c["write_kib"])
METRIC = "decode HBM GB/s + µs/call; prefill TFLOP/s (bf16) vs MI355X roofline"


def decode_workload(dev, seed=0):
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
    kv = int(sum(2 * int(m) * h * e * 2 for m in lens))
    io = 2 * n * h * e * 2 + int(sum(-(-int(m) // page) for m in lens)) * 4 + n * 4
    return dict(n=n, h=h, e=e, page=page, lens=lens, table=table, kc=kc, vc=vc, q=q,
                seqlens=seqlens, bytes=kv + io)


def timed(fn, steps, warmup):
    """Runs fn warmup + steps times; returns (wall seconds over the timed steps,
    per-step event milliseconds)."""
    for _ in range(warmup):
        fn()
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
          for _ in range(steps)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for a, b in ev:
        a.record()
        fn()
        b.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    return wall, [a.elapsed_time(b) for a, b in ev]


def cpu_decode_baseline(w, budget_s=4.0):
    """The C port of the reference's CPU decode on the host's physical cores, on the
    first sequences of the same batch (about 1/8 of its K/V)."""
    from cpu_attention import _kernel as K
    from oracle import cport

    ns = 8
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
        if time.perf_counter() - t0 >= budget_s or reps >= 50:
            break
    dt = (time.perf_counter() - t0) / reps
    nbytes = sum(2 * int(m) * h * e * 2 for m in lens) + 2 * ns * h * e * 2
    return {"value": round(nbytes / dt / 1e9, 3), "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": f"C port (oracle/ca_oracle.c, OpenMP) of the reference's paged decode on the "
                      f"first {ns} of the 64 sequences ({nbytes / 1e6:.0f} MB of K/V, bf16), "
                      f"{reps} calls, {dt * 1e3:.2f} ms/call"}


def cpu_prefill_baseline(budget_s=4.0):
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
        if time.perf_counter() - t0 >= budget_s or reps >= 20:
            break
    dt = (time.perf_counter() - t0) / reps
    flop = 4 * b * h * e * L * (L + 1) / 2
    return {"value": round(flop / dt / 1e12, 4), "unit": "TFLOP/s", "cores": threads, "kind": "port",
            "sample": f"C port of the reference's prefill, one (batch, head) of the config "
                      f"(L=S=4096 E=128 causal bf16), {reps} calls, {dt * 1e3:.1f} ms/call"}


def prefill_workload(dev):
    N, L, H, E = 4, 4096, 32, 128
    g = torch.Generator(device=dev).manual_seed(1)
    qkv = torch.randn(N * L, 3 * H * E, generator=g, device=dev).to(torch.bfloat16)
    q, k, v = (qkv[:, i * H * E:(i + 1) * H * E].view(N, L, H, E) for i in range(3))
    return qkv, q, k, v


def profile_pass(dev, mod, rt):
    src = torch.ones(COPY_BYTES // 4, dtype=torch.float32, device=dev)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    dst.copy_(src)
    torch.cuda.synchronize()
    del src, dst
    w = decode_workload(dev)
    out = torch.empty_like(w["q"])
    assert mod.decode(rt, w["q"], w["kc"], w["vc"], None, None, None, w["seqlens"], w["table"],
                      None, out) is not None
    torch.cuda.synchronize()
    del w, out
    torch.cuda.empty_cache()
    qkv, q, k, v = prefill_workload(dev)
    r = mod.flash(rt, q, k, v, None, True, 0, 0)
    assert r is not None and not isinstance(r, int)
    torch.cuda.synchronize()
    print("profile pass done", flush=True)


def main():
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    # The chip takes ~25 ms of continuous work to reach its operating clock (first
    # prefill calls 800 -> 565 us); the defaults warm up past that and time a
    # steady-state window (~35 ms decode, ~55 ms prefill).
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=300)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-prefill", action="store_true", help="skip the prefill line")
    ap.add_argument("--profile-pass", action="store_true",
                    help="no timing: one 1 GiB device copy, one decode call and one prefill call "
                         "(for rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE runs)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: the ops run within one device and this build "
              "has no multi-GPU path (see DESIGN.md for how it would shard). Use --gpus 1.",
              file=sys.stderr)
        sys.exit(2)

    from cpu_attention import _kernel as K

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    mod, rt = K.module(), K.runtime()
    K.set_host_checks(False)  # no host reads inside the timed loop

    if args.profile_pass:
        profile_pass(dev, mod, rt)
        return

    w = decode_workload(dev)
    out = torch.empty_like(w["q"])

    def step():
        r = mod.decode(rt, w["q"], w["kc"], w["vc"], None, None, None, w["seqlens"], w["table"],
                       None, out)
        assert r is not None

    wall, ms = timed(step, args.steps, args.warmup)
    call_ms = float(np.mean(ms))
    gbs_kernel = w["bytes"] / (call_ms * 1e-3) / 1e9
    value = w["bytes"] * args.steps / wall / 1e9
    res = {
        "metric": METRIC, "value": round(value, 2), "unit": "GB/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(wall / args.steps * 1e3, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": "paged decode flash_attn_with_kvcache bf16 N=64 H=32 E=128 page=32 "
                               "cache_seqlens U[17,2047] random-permutation page_table, no append",
                   "global_batch": w["n"], "seq_len": "17..2047", "parallelism": "none (1 GPU)"},
        "us_per_call": round(call_ms * 1e3, 2),
        "us_per_call_median": round(float(np.median(ms)) * 1e3, 2),
        "roofline": {"bound": "hbm", "achieved": round(gbs_kernel, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(gbs_kernel / HBM_PEAK_GBS, 4),
                     "traffic": traffic_bytes("decode"),
                     "kernel": "decode_tiles_kernel<128,bf16> (one call: rows of up to 2048 keys merge in-block)",
                     "algorithmic_bytes": w["bytes"]},
    }
    del w
    torch.cuda.empty_cache()

    if not args.no_prefill:
        N, L, H, E = 4, 4096, 32, 128
        qkv, q, k, v = prefill_workload(dev)

        def pstep():
            r = mod.flash(rt, q, k, v, None, True, 0, 0)
            assert r is not None and not isinstance(r, int)

        psteps, pwarm = max(3, args.steps // 2), max(3, args.warmup // 3)
        pwall, pms = timed(pstep, psteps, pwarm)
        flop = 4 * N * H * E * L * (L + 1) / 2
        pcall = float(np.mean(pms))
        tf = flop / (pcall * 1e-3) / 1e12
        res["prefill"] = {
            "workload": "flash_attn_func bf16 causal N=4 L=S=4096 H=32 E=128, q/k/v strided "
                        "chunks of a fused [N*L, 3*H*E] projection",
            "value": round(flop * len(pms) / pwall / 1e12, 2), "unit": "TFLOP/s",
            "steps": psteps, "warmup": pwarm,
            "us_per_call": round(pcall * 1e3, 1), "us_per_call_median": round(float(np.median(pms)) * 1e3, 1),
            "roofline": {"bound": "mfma", "achieved": round(tf, 1), "peak": BF16_PEAK_TFLOPS,
                         "unit": "TFLOP/s", "frac": round(tf / BF16_PEAK_TFLOPS, 4),
                         "traffic": traffic_bytes("prefill"), "kernel": "flash_bf16_p64_kernel<128>",
                         "algorithmic_flop": flop},
        }
        del qkv, q, k, v
        torch.cuda.empty_cache()

    if not args.no_cpu:
        w = decode_workload(dev)
        res["cpu_baseline"] = cpu_decode_baseline(w)
        del w
        if not args.no_prefill:
            res["prefill"]["cpu_baseline"] = cpu_prefill_baseline()
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
