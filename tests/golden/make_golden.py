"""Writes the golden fixtures in this directory from the CPU oracle.

    python tests/golden/make_golden.py

The reference ships no stored vectors for this path (its tests compare against a
float64 oracle at test time), so these fixtures are the oracle's outputs on
small seeded inputs, frozen: GPU tests compare the kernels with them without
recomputing anything, and a CPU test regenerates them and checks nothing drifted.
Each file is a numpy ``.npz`` (no pickles): inputs as exact bit patterns (bf16 as
uint16, fp32 as float32) and the float64 expected output or the expected cache
words.
"""

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

from oracle import bf16, layout  # noqa: E402
from oracle.attention import attention  # noqa: E402


def _bits(rng, shape, dtype):
    x = rng.standard_normal(shape).astype(np.float32)
    return bf16.from_float(x) if dtype == "bf16" else x


def _vals(bits, dtype):
    return (bf16.to_float(bits) if dtype == "bf16" else bits).astype(np.float64)


def flash_case(name, seed, b, sq, sk, h, d, dtype, causal, scale):
    rng = np.random.default_rng(seed)
    q, k, v = (_bits(rng, (b, n, h, d), dtype) for n in (sq, sk, sk))
    out = attention(_vals(q, dtype), _vals(k, dtype), _vals(v, dtype), scale, causal)
    return name, dict(kind="flash", dtype=dtype, causal=causal, scale=scale, q=q, k=k, v=v, out=out)


def decode_case(name, seed, lens, h, d, page, dtype, scale):
    rng = np.random.default_rng(seed)
    words = layout.words_per_token(d, dtype)
    npages = [-(-n // page) for n in lens]
    nb = sum(npages) + 1
    order = rng.permutation(nb)
    table = np.full((len(lens), max(npages) + 1), order[-1], np.int32)
    start = 0
    for i, n in enumerate(npages):
        table[i, :n] = order[start:start + n]
        start += n
    nan = bf16.from_float(np.array([np.nan], np.float32))[0] if dtype == "bf16" else np.float32(np.nan)
    cache = np.full((nb, h, page, d), nan)
    kc = layout.words_of(cache, dtype).reshape(nb, h, page * words).copy()
    vc = kc.copy()
    for i, n in enumerate(lens):
        key = layout.words_of(_bits(rng, (n, h, d), dtype), dtype)
        value = layout.words_of(_bits(rng, (n, h, d), dtype), dtype)
        layout.store(kc, vc, key, value, layout.prompt_slots(0, n, table[i], page), page)
    q = _bits(rng, (len(lens), h, d), dtype)
    out = layout.decode(_vals(q, dtype), kc, vc, table, lens, scale, page, dtype)
    return name, dict(kind="decode", dtype=dtype, scale=scale, page=page, q=q, kc=kc, vc=vc,
                      table=table, lens=np.asarray(lens, np.int32), out=out)


def store_case(name, seed, t, h, d, page, nb, dtype):
    rng = np.random.default_rng(seed)
    words = layout.words_per_token(d, dtype)
    slots = rng.permutation(nb * page)[:t].astype(np.int64)
    slots[::5] = -1
    key, value = (_bits(rng, (t, h, d), dtype) for _ in range(2))
    kc = np.zeros((nb, h, page * words), np.uint32)
    vc = np.zeros_like(kc)
    layout.store(kc, vc, layout.words_of(key, dtype), layout.words_of(value, dtype), slots, page)
    return name, dict(kind="store", dtype=dtype, page=page, key=key, value=value, slots=slots,
                      kc=kc, vc=vc)


CASES = [
    lambda: flash_case("flash_bf16_causal", 1, 1, 37, 70, 2, 64, "bf16", True, 64 ** -0.5),
    lambda: flash_case("flash_fp32_noncausal", 2, 2, 20, 33, 3, 32, "fp32", False, 0.2),
    lambda: flash_case("flash_fp32_causal_rows_empty", 3, 1, 40, 9, 1, 128, "fp32", True, 128 ** -0.5),
    lambda: decode_case("decode_bf16_p16", 4, [0, 1, 17, 100], 2, 64, 16, "bf16", 64 ** -0.5),
    lambda: decode_case("decode_fp32_p48", 5, [300, 47, 49], 3, 32, 48, "fp32", 0.5 * 32 ** -0.5),
    lambda: decode_case("decode_bf16_p32_e128", 6, [257, 33], 2, 128, 32, "bf16", 128 ** -0.5),
    lambda: store_case("store_bf16_p16", 7, 40, 2, 64, 16, 6, "bf16"),
    lambda: store_case("store_fp32_p32", 8, 50, 3, 32, 32, 4, "fp32"),
]


def generate():
    return dict(c() for c in CASES)


def main():
    for name, arrays in generate().items():
        np.savez_compressed(os.path.join(HERE, name + ".npz"), **{k: np.asarray(v) for k, v in arrays.items()})
        print(name)


if __name__ == "__main__":
    main()
