"""CPU address check of the flash kernels (tests/geom_check.hip): for every shape of
the GPU tests' grid, the BASELINE configs and a seeded random sample over tensor
layouts, the launcher's plan and the kernels' own index arithmetic are replayed on
the host, and every global access (buffer windows of the tile loads, Q rows,
guarded loads, output rows, workspace slots) and every direct-to-LDS tile load must
stay inside its tensor or buffer.  A planted mistake (partial key tiles' windows one
row too wide) must be caught."""

import os
import random
import shutil
import subprocess

import pytest
from route_cases import SEEDS as ROUTE_SEEDS, route_case

HERE = os.path.dirname(os.path.abspath(__file__))
SRC = os.path.join(HERE, "geom_check.hip")

pytestmark = pytest.mark.skipif(shutil.which("hipcc") is None, reason="hipcc is not on PATH")


@pytest.fixture(scope="module")
def checker(tmp_path_factory):
    exe = str(tmp_path_factory.mktemp("geom") / "geom_check")
    r = subprocess.run(["hipcc", "-x", "hip", "--offload-arch=gfx950", "-O1", "-std=c++17", "-w", SRC, "-o", exe],
                       capture_output=True, text=True, timeout=600)
    assert r.returncode == 0, r.stderr[-3000:]
    return exe


def strides(layout, b, n, h, e, fused_of=None):
    """Element strides (batch, token, head) of a [b, n, h, e] view."""
    if layout == "bshe":
        return (n * h * e, h * e, e)
    if layout == "fused":  # a q/k/v chunk of a [b * n, 3 * h * e] projection
        return (n * 3 * h * e, 3 * h * e, e)
    if layout == "bhse":  # a head-major tensor viewed as [b, n, h, e]
        return (h * n * e, e, n * e)
    if layout == "padded":  # token rows padded by 8 elements, batches by 64 tokens
        return ((n + 64) * (h * e + 8), h * e + 8, e)
    raise ValueError(layout)


def line(e, bf16, causal, b, sq, sk, h, layout="bshe"):
    qs = strides(layout, b, sq, h, e)
    ks = strides(layout, b, sk, h, e)
    return " ".join(str(x) for x in (e, int(bf16), int(causal), b, sq, sk, h, *qs, *ks, *ks))


def shapes():
    out = []
    lengths = [(1, 1), (17, 17), (64, 64), (129, 129), (1, 300), (100, 37), (37, 100), (257, 513)]
    for bf16 in (False, True):
        for e in (32, 64, 128):
            for sq, sk in lengths:
                for h in (1, 8):
                    for causal in (False, True):
                        out.append(line(e, bf16, causal, 1, sq, sk, h))
            # causal schedules, split keys, whole-block safe passes, pairs
            for b, sq, sk, h in [(1, 600, 600, 130), (1, 400, 400, 8), (1, 2048, 2048, 32), (2, 700, 1200, 48),
                                 (1, 2048, 4096, 32), (1, 1024, 1024, 16), (1, 64, 4096, 8), (2, 48, 8192, 16),
                                 (1, 128, 8192, 32), (1, 256, 8192, 32), (1, 1536, 1536, 2), (1, 1536, 1536, 44),
                                 (1, 600, 1536, 2), (1, 600, 1536, 86), (1, 512, 512, 130), (2, 300, 700, 2),
                                 (3, 77, 1000, 5), (1, 12, 4096, 32), (8, 9, 2048, 32), (1, 5, 4096, 32)]:
                for causal in (False, True):
                    out.append(line(e, bf16, causal, b, sq, sk, h))
    # the short-key route's GPU tests: layouts, partial blocks, the route's limits
    for b, sq, sk, h in [(1, 128, 128, 16), (2, 5, 128, 3), (1, 200, 37, 4), (3, 33, 97, 2), (1, 64, 1, 8),
                         (2, 31, 64, 5), (1, 96, 32, 1), (8, 128, 128, 32), (8, 129, 128, 32), (2, 32, 129, 4)]:
        for e in (32, 64, 128):
            for causal in (False, True):
                for lay in ("bshe", "fused", "bhse"):
                    out.append(line(e, True, causal, b, sq, sk, h, lay))
    # the short-key route past 128 keys, and the row-block limits its LDS sets
    for b, sq, sk, h in [(1, 256, 256, 16), (8, 256, 256, 16), (2, 129, 129, 3), (1, 200, 255, 4), (3, 37, 193, 2),
                         (4, 512, 256, 8), (2, 256, 256, 32), (3, 256, 256, 32), (3, 160, 160, 32)]:
        for e in (32, 64, 128):
            for causal in (False, True):
                for lay in ("bshe", "fused", "bhse"):
                    out.append(line(e, True, causal, b, sq, sk, h, lay))
    # a token stride whose 256 rows pass 2^32 bytes (64 rows stay under 2^31): the
    # short-key route's 32-bit offsets do not fit, so the call goes tiled
    big = 12 << 20
    out.append(" ".join(str(x) for x in (64, 1, 1, 1, 200, 200, 2, 200 * big, big, 64, 200 * big, big, 64,
                                          200 * big, big, 64)))
    # calls with keys under twice the rows that split (few query blocks)
    for e in (64, 128):
        for b, sq, sk, h in [(1, 4096, 4096, 4), (1, 2048, 2048, 12), (1, 1024, 1024, 8), (1, 3000, 3000, 8),
                             (1, 1500, 2100, 16), (1, 4096, 4096, 8), (1, 8192, 8192, 4), (2, 600, 600, 8),
                             (1, 768, 768, 4), (1, 512, 512, 8), (1, 1000, 1000, 2)]:
            for causal in (False, True):
                out.append(line(e, True, causal, b, sq, sk, h, "fused"))
    # single-row calls on the packed-heads route (split keys, merge counters)
    for b, sq, sk, h in [(8, 1, 2048, 32), (8, 1, 8192, 32), (2, 1, 16384, 16), (32, 1, 2048, 32), (64, 1, 512, 32),
                         (1, 1, 100000, 16), (3, 1, 77, 8)]:
        for e in (32, 64, 128):
            for bf16 in (False, True):
                for lay in ("bshe", "fused"):
                    out.append(line(e, bf16, False, b, sq, sk, h, lay))
    # the GPU route sweep's shapes (test_flash_gpu.py::test_route_sweep)
    for seed in range(ROUTE_SEEDS):
        b, sq, sk, h, e, dt, causal, lay = route_case(seed)
        out.append(line(e, dt == "bf16", causal, b, sq, sk, h, lay))
    # fp32 few-rows calls of 12 to 16 rows over 256 (batch, head) pairs (4 and 8 rows per wave)
    for b, sq, sk, h in [(4, 13, 100, 64), (4, 16, 2000, 64), (4, 14, 4096, 64), (2, 12, 700, 128), (16, 16, 4096, 32)]:
        for e in (32, 64, 128):
            for causal in (False, True):
                out.append(line(e, False, causal, b, sq, sk, h))
    # BASELINE: cfg1, cfg4 (fused q/k/v) and its cross shape
    out.append(line(64, True, True, 1, 128, 128, 16))
    out.append(line(128, True, True, 4, 4096, 4096, 32, "fused"))
    out.append(line(32, True, False, 8, 1, 2048, 32))
    rng = random.Random(7)
    for _ in range(300):
        e = rng.choice([32, 64, 128])
        bf16 = rng.random() < 0.6
        b = rng.choice([1, 2, 3])
        h = rng.choice([1, 2, 3, 8, 16, 33])
        sq = rng.choice([1, 2, 3, 4, 5, 8, 9, 16, 17, 31, 63, 64, 65, 127, 128, 129, 255, 256, 257, 300, 511, 700,
                         1024, 1100])
        sk = rng.choice([1, 2, 17, 63, 64, 65, 100, 255, 256, 257, 512, 513, 1000, 2047, 2048, 2049, 3000])
        out.append(line(e, bf16, rng.random() < 0.5, b, sq, sk, h, rng.choice(["bshe", "fused", "bhse", "padded"])))
    return out


def run(exe, lines, *args):
    return subprocess.run([exe, *args], input="\n".join(lines) + "\n", capture_output=True, text=True, timeout=600)


def test_every_access_inside_its_tensor(checker):
    lines = shapes()
    r = run(checker, lines)
    assert r.returncode == 0 and r.stdout.startswith("ok"), r.stdout[-2000:] + r.stderr[-2000:]
    n, accesses = map(int, r.stdout.split()[1:3])
    assert n == len(lines) and accesses > 10 ** 8


def test_a_planted_window_mistake_is_caught(checker):
    # partial key tiles (257 rows over 513 keys) with windows one row too wide
    r = run(checker, [line(64, True, True, 1, 257, 513, 8), line(128, True, False, 1, 300, 700, 2)], "--plant")
    assert r.returncode == 1 and "outside" in r.stdout, r.stdout
