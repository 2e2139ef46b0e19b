"""Seeded flash_attn_func shapes weighted toward the prefill's route boundaries:
short key ranges (the short-key kernel's 256-key limit), few query blocks over
long keys (the split rules), a few query rows (the few-rows routes), and general
shapes.  Used by the GPU parity sweep and by the CPU address check, so every shape
the sweep runs is also replayed on the host."""

import random

SEEDS = 200  # cases in the GPU sweep, all of them address-checked


def route_case(seed):
    """(batch, seq_q, seq_k, heads, head_dim, dtype ('bf16' | 'f32'), causal, layout)."""
    r = random.Random(seed * 7919 + 17)
    reg = r.random()
    e = r.choice([32, 64, 128])
    if reg < 0.35:  # short keys, either side of 256
        sk = r.randint(1, 260)
        sq = r.choice([r.randint(1, 64), r.randint(1, 600)])
        b, h = r.randint(1, 8), r.randint(1, 40)
        dt = "bf16" if r.random() < 0.85 else "f32"
    elif reg < 0.6:  # few query blocks over long keys
        sq = r.randint(700, 4300)
        sk = r.choice([sq, r.randint(sq // 2, 2 * sq), r.randint(900, 9000)])
        b, e = r.choice([1, 1, 2]), r.choice([64, 128])
        dt = "bf16" if r.random() < 0.8 else "f32"
        nqb = -(-sq // 256)
        h = max(1, min(48, r.randint(48, 140) // (b * nqb)))
    elif reg < 0.8:  # a few query rows
        sq, sk = r.randint(1, 16), r.randint(1, 9000)
        b, h = r.randint(1, 8), r.randint(1, 48)
        dt = "bf16" if r.random() < 0.7 else "f32"
    else:
        sq, sk = r.randint(1, 1500), r.randint(1, 1500)
        b, h = r.randint(1, 3), r.randint(1, 12)
        dt = "bf16" if r.random() < 0.6 else "f32"
    layout = r.choice(["bshe", "fused", "bhse"])
    if layout == "fused" and sq != sk:
        layout = "bshe"
    return b, sq, sk, h, e, dt, r.random() < 0.5, layout
