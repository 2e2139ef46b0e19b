"""Markdown tables from benchmarks/bench.py JSON files.

    python cpu-attention_amd/benchmarks/report.py out.json [more.json ...]

One table per kind (prefill, paged decode, store): per row the device-time
median (min-max) in µs, the API wall clock, the achieved rate against the
MI355X roofline, for prefill the ratio to torch SDPA's fused kernels, and with
``bench.py --counters`` the rocprofv3 columns (kernel time, HBM bytes against the
algorithmic ones, MFMA busy for prefill).
"""

import argparse
import json


def label(kind, shape):
    """A row's shape in SDPA's legend: N batch, L query length, S key/value length,
    H heads, E head dim (the reference's benchmarks/report.py:10-19).  Prefill rows
    mark `causal`; decode rows store the new token's K/V in the call unless marked
    `no append`."""
    n, s, h, e, flag = shape[:5]
    if kind == "flash":
        lq = shape[5] if len(shape) > 5 else s
        return f"N={n} L={lq} S={s} H={h} E={e}" + (" causal" if flag else "")
    s = f"{min(s)}..{max(s)}" if isinstance(s, list) else s
    return f"N={n} L=1 S={s} H={h} E={e}" + ("" if flag else " no append")


def us(t):
    return f"{t:,.0f}" if t >= 100 else f"{t:.1f}"


def spread(t):
    return f"{us(t['median'])} ({us(t['min'])}-{us(t['max'])})"


def tables(run):
    e = run["environment"]
    out = [f"{e['gpu']}, `{e['git']}`, torch {e['torch']} (HIP {e['hip']}); {e['library']}; "
           f"host checks {e.get('host_checks', 'on')}.\n"]
    for kind, title in (("flash", "Prefill, `flash_attn_func`"), ("paged", "Paged decode, `flash_attn_with_kvcache`"),
                        ("store", "`reshape_and_cache`")):
        rows = [x for x in run["rows"] if x["kind"] == kind]
        if not rows:
            continue
        rate = "TFLOP/s (of MFMA peak) | GB/s" if kind == "flash" else "GB/s (of 8 TB/s)"
        extra = " | SDPA gpu µs | ours / SDPA" if kind == "flash" else ""
        counted = any("counters" in x for x in rows)
        if counted:
            extra += " | rocprof kernel µs | HBM MB (x algorithmic)" + (" | MFMA busy" if kind == "flash" else "")
        ncols = (4 if kind == "flash" else 1) + ((3 if kind == "flash" else 2) if counted else 0)
        out += [f"**{title}**\n", f"| row | dtype | gpu µs, median (min-max) | API µs | {rate}{extra} |",
                "|---|---|---:|---:|" + "---:|" * ncols]
        for x in rows:
            t = x["timing"][x["ours"]]
            name = x["name"] if x["name"].startswith("cfg") else label(x["kind"], x["shape"])
            if x["name"].startswith("cfg"):
                name += f" ({label(x['kind'], x['shape'])})" if kind != "store" else ""
            val = x.get("tflops", x.get("gbs"))
            cell = f"{val:,.1f} ({x['roofline']['frac']:.1%})"
            if kind == "flash":
                cell += f" | {x['gbs']:,.0f}" if "gbs" in x else " | -"
            line = f"| {name} | {x['dtype']} | {spread(t['gpu'])} | {us(t['api']['median'])} | {cell}"
            if kind == "flash":
                if x.get("ref"):
                    line += f" | {us(x['timing'][x['ref']]['gpu']['median'])} | **{x['ratio']:.2f}**"
                else:
                    line += " | - | -"
            if counted:
                c = x.get("counters", {})
                work = x["gbs"] * t["gpu"]["median"] * 1e-6 * 1e9 if "gbs" in x else None
                line += f" | {c['kernel_us']:.1f}" if "kernel_us" in c else " | -"
                if "hbm_bytes" in c:
                    line += f" | {c['hbm_bytes'] / 1e6:,.1f}" + (f" ({c['hbm_bytes'] / work:.2f}x)" if work else "")
                else:
                    line += " | -"
                if kind == "flash":
                    line += f" | {c['mfma_util_pct']:.1f}%" if "mfma_util_pct" in c else " | -"
            out.append(line + " |")
        out.append("")
    return "\n".join(out)


def main():
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("files", nargs="+")
    args = ap.parse_args()
    for f in args.files:
        print(tables(json.load(open(f))))


if __name__ == "__main__":
    main()
