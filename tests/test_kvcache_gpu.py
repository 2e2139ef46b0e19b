"""flash_attn_with_kvcache (paged decode), the append, and reshape_and_cache on the
GPU against the float64 oracle and the layout oracle.  Mirrors the reference's
tests/test_kvcache.py case for case, then adds byte-level cache checks, the
engine entry (slots + out=), and the BASELINE decode shapes."""

import random
import threading

import numpy as np
import pytest
import torch

from cpu_attention import _kernel as K
from cpu_attention import flash_attn_with_kvcache, reshape_and_cache
from helpers import (NAME, appended, assert_close, attention, cache_words, layout, reference, row_words,
                     stage, values)

pytestmark = pytest.mark.gpu
DTYPES = [torch.float32, torch.bfloat16]


def decode(lens, h, d, page, dtype, seed, device, scale=None):
    q, kc, vc, bt, ks, vs = stage(lens, h, d, page, dtype, seed, device)
    seqlens = torch.tensor(lens, dtype=torch.int32, device=device)
    out = flash_attn_with_kvcache(q, kc, vc, cache_seqlens=seqlens, page_table=bt,
                                  softmax_scale=scale)
    assert_close(out, reference(q, ks, vs, scale or d ** -0.5), dtype, paged=True)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("page", [16, 32, 48, 64])
@pytest.mark.parametrize("d", [32, 64, 128])
@pytest.mark.parametrize("h", [1, 8])
def test_decode(cuda, dtype, page, d, h):
    decode([0, 1, page - 1, page, page + 1, 255, 257], h, d, page, dtype, seed=page + d, device=cuda)


@pytest.mark.parametrize("dtype", DTYPES)
def test_append_one_token(cuda, dtype):
    """k/v of one new token are written at cache_seqlens and attended in the same call."""
    lens, h, d = [5, 31, 64, 300], 8, 64
    q, kc, vc, bt, ks, vs = stage(lens, h, d, 16, dtype, seed=3, device=cuda)
    kn, vn = (torch.randn(len(lens), 1, h, d).to(dtype).to(cuda) for _ in range(2))
    seqlens = torch.tensor(lens, dtype=torch.int32, device=cuda)
    out = flash_attn_with_kvcache(q, kc, vc, k=kn, v=vn, cache_seqlens=seqlens, page_table=bt)
    ref = reference(q, *appended(ks, vs, kn, vn), d ** -0.5)
    assert_close(out, ref, dtype, paged=True)
    # flash-attn 2's name for the page table
    again = flash_attn_with_kvcache(q, kc, vc, cache_seqlens=seqlens + 1, block_table=bt)
    assert_close(again, ref, dtype, paged=True)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("nseqs", [2, 128, 129, 600])
def test_append_either_side_of_the_fused_limit(cuda, dtype, nseqs):
    """One token appended per sequence, over 16 and 128 x 8 = 1024 rows inside the
    decode kernel, over 129 x 8 = 1032 and 4800 rows by the store kernel first: the
    cache holds the bytes the layout oracle says (the unwritten slots keep their NaN
    poison) and the output attends the new token.  Edge positions: an empty row, the
    last slot of a page, the first slot of a new page, and a row past one block's
    2048 keys, whose blocks meet in the combine kernel."""
    h, d, page = 8, 64, 16
    rng = random.Random(nseqs)
    lens = [rng.randrange(0, 300) for _ in range(nseqs)]
    edge = [0, 15, 16, 2100][:nseqs]
    lens[:len(edge)] = edge
    # Stage one token more than lens, so that position lens[s] lies in a page of
    # sequence s (the helper points every row's page-table padding at one shared
    # block); the append overwrites that token.
    q, kc, vc, bt, ks, vs = stage([n + 1 for n in lens], h, d, page, dtype, seed=nseqs, device=cuda)
    ks, vs = [k[:, :n] for k, n in zip(ks, lens)], [v[:, :n] for v, n in zip(vs, lens)]
    kw, vw = cache_words(kc), cache_words(vc)
    g = torch.Generator().manual_seed(7)
    kn, vn = (torch.randn(nseqs, 1, h, d, generator=g).to(dtype).to(cuda) for _ in range(2))
    seqlens = torch.tensor(lens, dtype=torch.int32, device=cuda)
    out = flash_attn_with_kvcache(q, kc, vc, k=kn, v=vn, cache_seqlens=seqlens, page_table=bt)
    assert_close(out, reference(q, *appended(ks, vs, kn, vn), d ** -0.5), dtype, paged=True)
    layout.store(kw, vw, row_words(kn[:, 0]), row_words(vn[:, 0]),
                 layout.append_slots(lens, bt.cpu().numpy(), page), page)
    np.testing.assert_array_equal(cache_words(kc), kw)
    np.testing.assert_array_equal(cache_words(vc), vw)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("d", [32, 64, 128])
@pytest.mark.parametrize("h", [3, 6])
@pytest.mark.parametrize("mode", ["append", "slots"])
def test_scatter_store_of_one_token_per_sequence(cuda, dtype, d, h, mode):
    """Past 1024 rows, a decode's one token per sequence is stored by the scatter
    kernel before the decode (one wave per token and head, four heads per block).
    Head counts of 3 and 6 leave the last group of four part-empty; every head dim;
    the append at lens, and the engine path's store at given slots (every 7th
    sequence's slot is -1: nothing stored, and it attends its cached keys).  The
    cache holds the bytes the layout oracle says (unwritten slots keep their NaN
    poison) and the output matches the float64 reference."""
    nseqs, page = -(-1100 // h), 16
    rng = random.Random(h * 1000 + d)
    lens = [rng.randrange(1, 40) for _ in range(nseqs)]
    lens[:3] = [1, 15, 16]
    q, kc, vc, bt, ks, vs = stage([n + 1 for n in lens], h, d, page, dtype, seed=h + d, device=cuda)
    ks, vs = [k[:, :n] for k, n in zip(ks, lens)], [v[:, :n] for v, n in zip(vs, lens)]
    kw, vw = cache_words(kc), cache_words(vc)
    g = torch.Generator().manual_seed(d)
    kn, vn = (torch.randn(nseqs, 1, h, d, generator=g).to(dtype).to(cuda) for _ in range(2))
    slots = layout.append_slots(lens, bt.cpu().numpy(), page)
    if mode == "append":
        seqlens = torch.tensor(lens, dtype=torch.int32, device=cuda)
        out = flash_attn_with_kvcache(q, kc, vc, k=kn, v=vn, cache_seqlens=seqlens, page_table=bt)
        ks2, vs2 = appended(ks, vs, kn, vn)
    else:
        skip = set(range(0, nseqs, 7))
        slots[sorted(skip)] = -1
        post = torch.tensor([n if s in skip else n + 1 for s, n in enumerate(lens)], dtype=torch.int32,
                            device=cuda)
        out = K.module().decode(K.runtime(), q, kc, vc, kn, vn, torch.from_numpy(slots).to(cuda), post, bt,
                                None, None)
        ks2 = [k if s in skip else torch.cat([k, kn[s:s + 1]], 1) for s, k in enumerate(ks)]
        vs2 = [v if s in skip else torch.cat([v, vn[s:s + 1]], 1) for s, v in enumerate(vs)]
    assert_close(out, reference(q, ks2, vs2, d ** -0.5), dtype, paged=True)
    layout.store(kw, vw, row_words(kn[:, 0]), row_words(vn[:, 0]), slots, page)
    np.testing.assert_array_equal(cache_words(kc), kw)
    np.testing.assert_array_equal(cache_words(vc), vw)


def long_tiles(rows, width, page, d, esize):
    """Whether the decode takes 256-key tiles (csrc/ca_decode.hip, decode_tile_keys):
    a page table of more than 512 keys and at most 2048, 256 rows or more, at most
    80 Mi K elements at capacity, rows of at most 128 bytes."""
    cap = width * page
    return 512 < cap <= 2048 and rows >= 256 and rows * cap * d <= 80 << 20 and d * esize <= 128


@pytest.mark.parametrize("dtype,d,tiles", [(dt, d, "short") for dt in DTYPES for d in (32, 64, 128)] +
                         [(torch.bfloat16, 32, "long"), (torch.bfloat16, 64, "long"), (torch.float32, 32, "long")])
def test_both_tile_sizes(cuda, dtype, d, tiles):
    """A batch on each side of the 64/256-key tile choice, with rows at the edges of
    tiles and of blocks (512 keys of 64-key tiles, 2048 of 256-key tiles) and rows
    that span several blocks and are merged: a one-token append attended in the same
    call, then a plain decode of the same cache.  256-key tiles serve only narrow
    rows (bf16 E <= 64, fp32 E = 32)."""
    page = 16
    if tiles == "short":
        h, lens = 2, [0, 63, 64, 511, 512, 513, 1100, 3000]
    else:
        h, rng = 8, random.Random(d)
        lens = [0, 255, 256, 1023, 1024, 2029, 2030] + [rng.randrange(0, 2031) for _ in range(57)]
    # staged with one token more than lens, so that position lens[s] lies in a page of
    # sequence s; the append overwrites that token
    q, kc, vc, bt, ks, vs = stage([n + 1 for n in lens], h, d, page, dtype, seed=d, device=cuda)
    esize = 2 if dtype == torch.bfloat16 else 4
    assert long_tiles(len(lens) * h, bt.shape[1], page, d, esize) == (tiles == "long")
    ks, vs = [k[:, :n] for k, n in zip(ks, lens)], [v[:, :n] for v, n in zip(vs, lens)]
    g = torch.Generator().manual_seed(d)
    kn, vn = (torch.randn(len(lens), 1, h, d, generator=g).to(dtype).to(cuda) for _ in range(2))
    seqlens = torch.tensor(lens, dtype=torch.int32, device=cuda)
    out = flash_attn_with_kvcache(q, kc, vc, k=kn, v=vn, cache_seqlens=seqlens, page_table=bt)
    ref = reference(q, *appended(ks, vs, kn, vn), d ** -0.5)
    assert_close(out, ref, dtype, paged=True)
    again = flash_attn_with_kvcache(q, kc, vc, cache_seqlens=seqlens + 1, page_table=bt)
    assert_close(again, ref, dtype, paged=True)


def test_fp32_rows_of_long_tiles(cuda):
    """fp32 rows of 1856 rows whose page tables span 192 keys.  On 256-key tiles, as
    this call then ran, a lane summed up to 64 keys of P.V in one fma chain, and the
    row of 81 keys (sequence 79, head 10) reached 1.11e-6 against the reference's
    1e-6 gate; the kernel now sums a lane's odd and even keys apart, and page tables
    of at most 512 keys take 64-key tiles.  These are that call's lengths, page size
    and staging seed (found by a randomized sweep)."""
    lens = [14, 93, 28, 25, 28, 71, 49, 39, 39, 47, 37, 23, 23, 91, 32, 31, 31, 61, 36, 57, 22, 49, 16, 12,
            73, 77, 100, 10, 27, 76, 16, 88, 8, 33, 84, 46, 41, 100, 68, 64, 55, 9, 47, 44, 50, 83, 49, 63, 38,
            93, 42, 82, 30, 14, 1, 46, 37, 37, 1, 57, 76, 97, 88, 26, 38, 6, 56, 56, 16, 0, 35, 25, 75, 92, 10,
            27, 17, 93, 90, 81, 60, 2, 98, 31, 23, 30, 19, 26, 98, 58, 9, 84, 56, 20, 93, 48, 23, 41, 41, 8,
            70, 29, 35, 38, 34, 36, 92, 72, 31, 42, 58, 73, 55, 50, 25, 52]
    decode(lens, 16, 64, 48, torch.float32, seed=137, device=cuda)


@pytest.mark.parametrize("host_checks", [True, False])
def test_uneven_lengths(cuda, host_checks):
    """Lopsided batches (the reference sweeps thread counts here; the GPU splits every
    row into 256-key tiles, so this sweeps the host-check mode instead)."""
    old = K.set_host_checks(host_checks)
    try:
        for seed, lens in enumerate(([0, 2047, 1, 17, 64], [2047, 16], [5, 3, 1024])):
            decode(lens, 8, 64, 16, torch.float32, seed=seed, device=cuda)
    finally:
        K.set_host_checks(old)


@pytest.mark.parametrize("dtype", DTYPES)
def test_fused_projection_strides(cuda, dtype):
    """q and the new k/v as chunks of one fused [b, 1, 3 h d] projection."""
    lens, h, d = [40, 200], 8, 64
    q, kc, vc, bt, ks, vs = stage(lens, h, d, 32, dtype, seed=4, device=cuda)
    qkv = torch.randn(len(lens), 1, 3 * h * d).to(dtype).to(cuda)
    qn, kn, vn = (qkv[..., i * h * d:(i + 1) * h * d].view(len(lens), 1, h, d) for i in range(3))
    out = flash_attn_with_kvcache(qn, kc, vc, k=kn, v=vn, page_table=bt,
                                  cache_seqlens=torch.tensor(lens, dtype=torch.int32, device=cuda))
    assert_close(out, reference(qn, *appended(ks, vs, kn, vn), d ** -0.5), dtype, paged=True)


@pytest.mark.parametrize("seed", range(30))
def test_fuzz(cuda, seed):
    r = random.Random(seed)
    lens = [r.randint(0, 1100) for _ in range(r.randint(1, 6))]
    d = r.choice([32, 64, 128])
    decode(lens, r.choice([1, 4, 12]), d, r.choice([16, 32, 48, 64]), r.choice(DTYPES), seed,
           cuda, scale=r.choice([1.0, 0.5]) * d ** -0.5)


def test_concurrent_callers(cuda):
    """Python threads calling at once each get their own correct result."""
    cases = [stage([100 + 50 * i, 33], 8, 64, 16, torch.float32, seed=i, device=cuda) for i in range(4)]
    refs = [reference(q, ks, vs, 0.125) for q, _, _, _, ks, vs in cases]
    errors = []

    def worker(i):
        q, kc, vc, bt, _, _ = cases[i]
        seqlens = torch.tensor([100 + 50 * i, 33], dtype=torch.int32, device=cuda)
        for _ in range(20):
            out = flash_attn_with_kvcache(q, kc, vc, cache_seqlens=seqlens, page_table=bt,
                                          softmax_scale=0.125)
            errors.append(float(np.abs(values(out) - refs[i]).max()))

    pool = [threading.Thread(target=worker, args=(i,)) for i in range(4)]
    for t in pool:
        t.start()
    for t in pool:
        t.join()
    assert len(errors) == 80 and max(errors) <= 1e-6


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("page", [16, 32])
def test_reshape_and_cache(cuda, dtype, page):
    """reshape_and_cache writes the same cache an append does (byte for byte);
    negative slots skip, and k/v may be chunks of a fused projection."""
    lens, h, d = [70, 5], 8, 64
    q, kc, vc, bt, ks, vs = stage(lens, h, d, page, dtype, seed=6, device=cuda)
    kc2, vc2 = torch.full_like(kc, float("nan")), torch.full_like(vc, float("nan"))
    kv = torch.cat([torch.cat([k[0], v[0]], -1) for k, v in zip(ks, vs)])  # [tokens, h, 2d]
    pos = torch.cat([torch.arange(n) for n in lens])
    seq = torch.cat([torch.full((n,), i) for i, n in enumerate(lens)])
    slots = bt.cpu()[seq, pos // page].long() * page + pos % page
    kv = torch.cat([kv, torch.randn(3, h, 2 * d).to(dtype).to(cuda)])  # 3 padding tokens, slot -1
    reshape_and_cache(kv[..., :d], kv[..., d:], kc2, vc2,
                      torch.cat([slots, torch.full((3,), -1, dtype=torch.int64)]).to(cuda))
    seqlens = torch.tensor(lens, dtype=torch.int32, device=cuda)
    out = flash_attn_with_kvcache(q, kc2, vc2, cache_seqlens=seqlens, page_table=bt)
    assert_close(out, reference(q, ks, vs, d ** -0.5), dtype, paged=True)
    np.testing.assert_array_equal(cache_words(kc2), cache_words(kc))
    np.testing.assert_array_equal(cache_words(vc2), cache_words(vc))


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("d", [32, 64, 128])
@pytest.mark.parametrize("page", [16, 48])
@pytest.mark.parametrize("pattern", ["consecutive", "scattered", "unaligned_run"])
def test_store_bit_exact(cuda, dtype, d, page, pattern):
    """The store against the layout oracle, whole cache compared as bytes (unwritten
    slots keep their NaN poison)."""
    g = torch.Generator().manual_seed(d * page)
    nb, h, T = 9, 3, 70
    cap = nb * page
    if pattern == "consecutive":
        slots = torch.arange(page, page + T)
    elif pattern == "scattered":
        slots = torch.randperm(cap, generator=g)[:T]
    else:
        slots = torch.arange(5, 5 + T)  # runs that start mid-page and cross pages
    slots = slots.clone()
    slots[::7] = -1  # padding
    # key/value as chunks of one fused [T, 3*h*d] projection: token stride 3*h*d
    src = torch.randn(T, 3 * h * d, generator=g).to(dtype).to(cuda)
    key, value = src[:, :h * d].view(T, h, d), src[:, 2 * h * d:].view(T, h, d)
    kc = torch.full((nb, h, page, d), float("nan"), dtype=dtype, device=cuda)
    vc = kc.clone()
    reshape_and_cache(key, value, kc, vc, slots.to(cuda))
    kw = cache_words(torch.full((nb, h, page, d), float("nan"), dtype=dtype))
    vw = kw.copy()
    layout.store(kw, vw, row_words(key), row_words(value), slots.numpy(), page)
    np.testing.assert_array_equal(cache_words(kc), kw)
    np.testing.assert_array_equal(cache_words(vc), vw)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("source", ["contiguous", "fused_view", "module_entry"])
def test_store_one_token(cuda, dtype, source):
    """One token (a batch-1 serving step): reshape_and_cache and the module's store
    entry, from a contiguous [1, H, E] tensor and from a one-token view of a fused
    projection, byte-equal to the layout oracle."""
    h, d, page, nb = 4, 128, 16, 5
    g = torch.Generator().manual_seed(3)
    fused = torch.randn(1, 3 * h * d, generator=g).to(dtype).to(cuda)
    if source == "fused_view":
        key, value = fused[:, :h * d].view(1, h, d), fused[:, 2 * h * d:].view(1, h, d)
    else:
        key, value = (torch.randn(1, h, d, generator=g).to(dtype).to(cuda) for _ in range(2))
    slots = torch.tensor([2 * page + 7], dtype=torch.int64)
    kc = torch.full((nb, h, page, d), float("nan"), dtype=dtype, device=cuda)
    vc = kc.clone()
    if source == "module_entry":
        assert K.module().store(K.runtime(), key, value, kc, vc, slots.to(cuda)) is True
    else:
        reshape_and_cache(key, value, kc, vc, slots.to(cuda))
    kw = cache_words(torch.full((nb, h, page, d), float("nan"), dtype=dtype))
    vw = kw.copy()
    layout.store(kw, vw, row_words(key), row_words(value), slots.numpy(), page)
    np.testing.assert_array_equal(cache_words(kc), kw)
    np.testing.assert_array_equal(cache_words(vc), vw)


@pytest.mark.parametrize("dtype", DTYPES)
def test_cache_batch_idx(cuda, dtype):
    """``cache_batch_idx`` picks the page-table row of each query
    (flash_attn_interface.py:103-104): here queries attend the staged sequences in
    another order, one of them twice."""
    lens, h, d, page = [40, 3, 77], 4, 64, 16
    q, kc, vc, bt, ks, vs = stage(lens, h, d, page, dtype, seed=17, device=cuda)
    idx = torch.tensor([2, 0, 2, 1])
    g = torch.Generator().manual_seed(4)
    q4 = torch.randn(4, 1, h, d, generator=g).to(dtype).to(cuda)
    seqlens = torch.tensor([lens[i] for i in idx], dtype=torch.int32, device=cuda)
    for where in (cuda, "cpu"):
        out = flash_attn_with_kvcache(q4, kc, vc, cache_seqlens=seqlens, page_table=bt,
                                      cache_batch_idx=idx.to(where))
        ref = reference(q4, [ks[i] for i in idx], [vs[i] for i in idx], d ** -0.5)
        assert_close(out, ref, dtype, paged=True)


@pytest.mark.parametrize("dtype", DTYPES)
def test_multi_token_append_bytes(cuda, dtype):
    """The multi-token append (flash_attn_interface.py:109-117) writes what the
    layout oracle's prompt slots say, then decodes over the grown cache."""
    h, d, page = 4, 64, 32
    nb = 12
    g = torch.Generator().manual_seed(11)
    table = torch.randperm(nb, generator=g)[:8].to(torch.int32).view(2, 4)
    kc = torch.full((nb, h, page, d), float("nan"), dtype=dtype, device=cuda)
    vc = kc.clone()
    k = torch.randn(2, 50, h, d, generator=g).to(dtype).to(cuda)
    v = torch.randn(2, 50, h, d, generator=g).to(dtype).to(cuda)
    q = torch.randn(2, 1, h, d, generator=g).to(dtype).to(cuda)
    start = torch.tensor([3, 40], dtype=torch.int32)
    kw = cache_words(kc.cpu())
    vw = kw.copy()
    for i in range(2):
        s = layout.prompt_slots(int(start[i]), 50, table[i].numpy(), page)
        layout.store(kw, vw, row_words(k[i]), row_words(v[i]), s, page)
    flash_attn_with_kvcache(q, kc, vc, k=k, v=v, cache_seqlens=start.to(cuda), page_table=table.to(cuda))
    np.testing.assert_array_equal(cache_words(kc), kw)
    np.testing.assert_array_equal(cache_words(vc), vw)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("q_rank", [3, 4])
def test_engine_entry_slots_and_out(cuda, dtype, q_rank):
    """The engine path (examples/ops.py:19-31): store each sequence's new token at
    ``slots`` (negative skips), lens is the post-store length, caller-owned out."""
    lens, h, d, page = [30, 64, 1], 4, 128, 16
    q, kc, vc, bt, ks, vs = stage(lens, h, d, page, dtype, seed=9, device=cuda)
    kn, vn = (torch.randn(len(lens), h, d).to(dtype).to(cuda) for _ in range(2))
    qn = q[:, 0] if q_rank == 3 else q
    pos = torch.tensor(lens)
    slots = bt.cpu()[torch.arange(3), pos // page].long() * page + pos % page
    slots[2] = -1  # sequence 2 stores nothing and attends its 1 cached key
    post = torch.tensor([31, 65, 1], dtype=torch.int32, device=cuda)
    out = torch.empty_like(qn)
    mod = K.module()
    kk, vv = (kn, vn) if q_rank == 3 else (kn[:, None], vn[:, None])
    got = mod.decode(K.runtime(), qn, kc, vc, kk, vv, slots.to(cuda), post, bt, None, out)
    assert got is out
    ks2 = [torch.cat([ks[0], kn[None, 0:1]], 1), torch.cat([ks[1], kn[None, 1:2]], 1), ks[2]]
    vs2 = [torch.cat([vs[0], vn[None, 0:1]], 1), torch.cat([vs[1], vn[None, 1:2]], 1), vs[2]]
    ref = reference(q, ks2, vs2, d ** -0.5)
    assert_close(out.view(ref.shape), ref, dtype, paged=True)
    # declines: slots without k/v, a wrong-dtype out
    assert mod.decode(K.runtime(), qn, kc, vc, None, None, slots.to(cuda), post, bt, None, None) is None
    assert mod.decode(K.runtime(), qn, kc, vc, kk, vv, slots.to(cuda), post, bt, None,
                      out.float() if dtype == torch.bfloat16 else out.bfloat16()) is None


def test_host_checks_off_never_faults(cuda):
    """Without the host read, out-of-range slots are not stored and lengths past the
    table are clamped to its capacity: no fault, finite output."""
    old = K.set_host_checks(False)
    try:
        h, d, page = 2, 64, 16
        kc = torch.zeros(4, h, page, d, device=cuda)
        vc = torch.zeros_like(kc)
        key = torch.randn(3, h, d, device=cuda)
        reshape_and_cache(key, key, kc, vc, torch.tensor([0, 10**6, -5], device=cuda))
        kflat = kc[0].reshape(h, -1)
        assert torch.equal(kflat[:, ::page], key[0])  # K word (d, t=0) sits at d*P
        assert torch.equal(vc[0, :, 0], key[0])
        assert int((kc != 0).sum()) == h * d and int((vc != 0).sum()) == h * d
        q = torch.randn(2, 1, h, d, device=cuda)
        bt = torch.tensor([[0, 1], [2, 3]], dtype=torch.int32, device=cuda)
        out = flash_attn_with_kvcache(q, kc, vc, cache_seqlens=torch.tensor([1000, 5], dtype=torch.int32,
                                                                            device=cuda), page_table=bt)
        assert torch.isfinite(out).all()
    finally:
        K.set_host_checks(old)


@pytest.mark.parametrize("nseqs", [4095, 4100])
def test_many_sequences(cuda, nseqs):
    """Thousands of short rows, many of them empty: one wave per 256-key tile of
    8190+ rows, single-tile rows written directly.  Every row checked."""
    h, d, page = 2, 32, 16
    rng = np.random.default_rng(nseqs)
    lens = rng.integers(0, 300, size=nseqs)
    lens[::97] = 0
    width = -(-int(lens.max()) // page)
    nb = nseqs * width
    table = torch.from_numpy(rng.permutation(nb).astype(np.int32)).view(nseqs, width)
    g = torch.Generator().manual_seed(nseqs)
    kc = torch.full((nb, h, page, d), float("nan"), dtype=torch.bfloat16, device=cuda)
    vc = torch.full_like(kc, float("nan"))
    total = int(lens.sum())
    key = torch.randn(total, h, d, generator=g).bfloat16()
    value = torch.randn(total, h, d, generator=g).bfloat16()
    slots = np.concatenate([layout.prompt_slots(0, int(m), table[i].numpy(), page)
                            for i, m in enumerate(lens)])
    reshape_and_cache(key.to(cuda), value.to(cuda), kc, vc, torch.from_numpy(slots).to(cuda))
    q = torch.randn(nseqs, 1, h, d, generator=g).bfloat16()
    out = flash_attn_with_kvcache(q.to(cuda), kc, vc, page_table=table.to(cuda),
                                  cache_seqlens=torch.from_numpy(lens.astype(np.int32)).to(cuda))
    starts = np.concatenate([[0], np.cumsum(lens)])
    kv, vv, qv = values(key), values(value), values(q)
    ref = np.zeros((nseqs, 1, h, d))
    for i, m in enumerate(lens):
        if m:
            ref[i] = attention(qv[i:i + 1], kv[None, starts[i]:starts[i + 1]],
                               vv[None, starts[i]:starts[i + 1]], d ** -0.5)[0]
    assert_close(out, ref, torch.bfloat16, paged=True)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("n", [2, 40, 100])
def test_prompt_append_in_one_call(cuda, dtype, n):
    """The prompt append (k/v with n new tokens per sequence) through the single
    native call: the cache bytes are what the layout oracle's prompt slots give,
    and q attends every old and new token."""
    lens, h, d, page = [0, 5, 31, 100], 4, 64, 16
    q, kc, vc, bt, ks, vs = stage(lens, h, d, page, dtype, seed=n, device=cuda)
    # Room for n more tokens: each sequence keeps its pages and gets fresh
    # (NaN-filled) blocks for the rest of a wider page table.
    cols = -(-(max(lens) + n) // page)
    nb, table = kc.shape[0], bt.cpu()
    rows = []
    for i, m in enumerate(lens):
        own = -(-m // page)
        fresh = torch.arange(nb, nb + cols - own, dtype=torch.int32)
        nb += cols - own
        rows.append(torch.cat([table[i, :own], fresh]))
    bt = torch.stack(rows).to(cuda)
    pad = torch.full((nb - kc.shape[0], *kc.shape[1:]), float("nan"), dtype=dtype, device=cuda)
    kc, vc = torch.cat([kc, pad]), torch.cat([vc, pad.clone()])
    g = torch.Generator().manual_seed(100 + n)
    kn, vn = (torch.randn(len(lens), n, h, d, generator=g).to(dtype).to(cuda) for _ in range(2))
    kw, vw = cache_words(kc), cache_words(vc)
    for i in range(len(lens)):
        s = layout.prompt_slots(lens[i], n, bt[i].cpu().numpy(), page)
        layout.store(kw, vw, row_words(kn[i]), row_words(vn[i]), s, page)
    seqlens = torch.tensor(lens, dtype=torch.int32, device=cuda)
    out = flash_attn_with_kvcache(q, kc, vc, k=kn, v=vn, cache_seqlens=seqlens, page_table=bt)
    np.testing.assert_array_equal(cache_words(kc), kw)
    np.testing.assert_array_equal(cache_words(vc), vw)
    ks2 = [torch.cat([a, kn[i:i + 1]], 1) for i, a in enumerate(ks)]
    vs2 = [torch.cat([a, vn[i:i + 1]], 1) for i, a in enumerate(vs)]
    assert_close(out, reference(q, ks2, vs2, d ** -0.5), dtype, paged=True)
    assert torch.equal(seqlens.cpu(), torch.tensor(lens, dtype=torch.int32))  # not mutated


def test_prompt_append_strided_and_cpu_lengths(cuda):
    """k/v as strided chunks of a fused projection and cache_seqlens as an int or
    a CPU tensor take the same single call."""
    h, d, page, n = 2, 32, 16, 20
    nb = 8
    table = torch.arange(nb, dtype=torch.int32).view(2, 4)
    kc = torch.zeros(nb, h, page, d, dtype=torch.bfloat16, device=cuda)
    vc = torch.zeros_like(kc)
    g = torch.Generator().manual_seed(7)
    kv = torch.randn(2, n, 3 * h * d, generator=g).bfloat16().to(cuda)
    k, v = (kv[..., i * h * d:(i + 1) * h * d].view(2, n, h, d) for i in (0, 2))
    q = torch.randn(2, 1, h, d, generator=g).bfloat16().to(cuda)
    out = flash_attn_with_kvcache(q, kc, vc, k=k, v=v, cache_seqlens=0, page_table=table.to(cuda))
    ref = reference(q, [k[0:1], k[1:2]], [v[0:1], v[1:2]], d ** -0.5)
    assert_close(out, ref, torch.bfloat16, paged=True)
    out2 = flash_attn_with_kvcache(q, kc, vc, cache_seqlens=torch.tensor([n, n], dtype=torch.int32),
                                   page_table=table)
    assert_close(out2, ref, torch.bfloat16, paged=True)


def test_prompt_append_past_the_page_table(cuda):
    """More new tokens than the page table holds: with host checks the reference's
    ValueError, raised before any token is written; without them no fault, the tokens that fit are stored and the
    row attends the table's capacity."""
    h, d, page = 2, 64, 16
    table = torch.tensor([[0, 1]], dtype=torch.int32, device=cuda)
    kc = torch.zeros(2, h, page, d, device=cuda)
    vc = torch.zeros_like(kc)
    k = torch.randn(1, 40, h, d, device=cuda)
    q = torch.randn(1, 1, h, d, device=cuda)
    with pytest.raises(ValueError):
        flash_attn_with_kvcache(q, kc, vc, k=k, v=k, cache_seqlens=torch.tensor([0], dtype=torch.int32,
                                                                                device=cuda),
                                page_table=table)
    torch.cuda.synchronize()
    assert not kc.any() and not vc.any(), "a refused prompt wrote part of itself"
    old = K.set_host_checks(False)
    try:
        out = K.module().append_decode(K.runtime(), q, kc, vc, k, k, torch.tensor([0], dtype=torch.int32,
                                                                                   device=cuda), table, None)
        assert out is not None and torch.isfinite(out).all()
        assert torch.equal(vc[0].permute(1, 0, 2).reshape(-1, h, d), k[0, :16])
        assert torch.equal(vc[1].permute(1, 0, 2).reshape(-1, h, d), k[0, 16:32])
        ref = attention(values(q[0:1]), values(k[:, :32]), values(k[:, :32]), d ** -0.5)
        assert np.abs(values(out) - ref).max() <= 1e-5
    finally:
        K.set_host_checks(old)
