"""The BASELINE decode workloads at full size on the GPU: cfg3 with every sequence
checked against the float64 oracle, cfg2 with every row, and cfg5's store + decode
loop with the cache bytes compared to the layout oracle after staging and after the
first and last steps (the pages each step appends to after every step)."""

import numpy as np
import pytest
import torch

from cpu_attention import _kernel as K
from cpu_attention import flash_attn_with_kvcache, reshape_and_cache
from helpers import assert_close, attention, cache_words, layout, row_words, values

pytestmark = pytest.mark.gpu


def paged_batch(n, h, e, page, lens, dtype, device, seed):
    """Caches filled with N(0,1) K/V for ``lens`` tokens per sequence, a random
    permutation page table (one pool of blocks, shuffled)."""
    g = torch.Generator(device=device).manual_seed(seed)
    width = -(-max(lens) // page)
    nb = n * width
    perm = torch.randperm(nb, generator=g, device=device).to(torch.int32)
    table = perm.view(n, width)
    kc = torch.randn(nb, h, page, e, generator=g, device=device).to(dtype)
    vc = torch.randn(nb, h, page, e, generator=g, device=device).to(dtype)
    return kc, vc, table


def dense_kv(kc, vc, table_row, length, page):
    """One sequence's K/V [len, H, E] as float64, read back through the layout oracle."""
    dtype = "bf16" if kc.dtype == torch.bfloat16 else "fp32"
    pages = -(-length // page)
    blocks = table_row[:pages].long()
    kw, vw = cache_words(kc[blocks]), cache_words(vc[blocks])
    k, v = layout.gather(kw, vw, np.arange(pages), length, page)
    return layout.to_values(k, dtype), layout.to_values(v, dtype)


def test_cfg3_decode_bf16_full_size(cuda):
    """N=64 H=32 E=128 page=32, lens U[17,2047], random-permutation page table, no
    append; the oracle checks every sequence (all heads)."""
    n, h, e, page = 64, 32, 128, 32
    rng = np.random.default_rng(3)
    lens = rng.integers(17, 2048, size=n)
    kc, vc, table = paged_batch(n, h, e, page, lens, torch.bfloat16, cuda, seed=3)
    q = torch.randn(n, 1, h, e, device=cuda).to(torch.bfloat16)
    seqlens = torch.tensor(lens, dtype=torch.int32, device=cuda)
    out = flash_attn_with_kvcache(q, kc, vc, cache_seqlens=seqlens, page_table=table)
    assert torch.isfinite(out).all()
    tcpu = table.cpu()
    for s in range(n):
        k, v = dense_kv(kc, vc, tcpu[s], int(lens[s]), page)
        ref = attention(values(q[s:s + 1]), k[None], v[None], e ** -0.5)
        assert_close(out[s:s + 1], ref, torch.bfloat16, paged=True)


def test_cfg2_decode_fp32_with_append(cuda):
    """N=8 H=16 E=64 page=16 fp32, lens U[17,2047], caches filled through
    reshape_and_cache, one new token appended per sequence; every row checked."""
    n, h, e, page = 8, 16, 64, 16
    rng = np.random.default_rng(2)
    lens = rng.integers(17, 2048, size=n)
    width = -(-(int(lens.max()) + 1) // page)
    nb = n * width
    g = torch.Generator().manual_seed(2)
    table = torch.randperm(nb, generator=g).to(torch.int32).view(n, width)
    kc = torch.full((nb, h, page, e), float("nan"), device=cuda)
    vc = torch.full_like(kc, float("nan"))
    ks = [torch.randn(int(m), h, e, generator=g) for m in lens]
    vs = [torch.randn(int(m), h, e, generator=g) for m in lens]
    slots = torch.cat([torch.from_numpy(layout.prompt_slots(0, int(m), table[i].numpy(), page))
                       for i, m in enumerate(lens)])
    reshape_and_cache(torch.cat(ks).to(cuda), torch.cat(vs).to(cuda), kc, vc, slots.to(cuda))
    q = torch.randn(n, 1, h, e, generator=g).to(cuda)
    kn, vn = (torch.randn(n, 1, h, e, generator=g).to(cuda) for _ in range(2))
    out = flash_attn_with_kvcache(q, kc, vc, k=kn, v=vn, page_table=table.to(cuda),
                                  cache_seqlens=torch.tensor(lens, dtype=torch.int32, device=cuda))
    ref = np.concatenate([
        attention(values(q[i:i + 1]), values(torch.cat([ks[i], kn[i].cpu()]))[None],
                  values(torch.cat([vs[i], vn[i].cpu()]))[None], e ** -0.5)
        for i in range(n)])
    assert_close(out, ref, torch.float32, paged=True)


def test_cfg5_store_and_decode_loop(cuda):
    """N=128 H=32 E=128 page=16 bf16: stage prompts of lengths U[64,1024] through
    reshape_and_cache with ~10% negative (padding) slots, then 32 decode steps each
    appending one token and attending.  Cache bytes equal the layout oracle after
    staging, the pages each step appends to after every step, and the whole caches
    after the first and last steps; sampled rows match the float64 oracle."""
    n, h, e, page, steps = 128, 32, 128, 16, 32
    rng = np.random.default_rng(5)
    lens = rng.integers(64, 1025, size=n)
    width = -(-(int(lens.max()) + steps) // page)
    nb = n * width
    table = torch.from_numpy(rng.permutation(nb).astype(np.int32)).view(n, width)
    slots = np.concatenate([layout.prompt_slots(0, int(m), table[i].numpy(), page)
                            for i, m in enumerate(lens)])
    # ~10% padding tokens (slot -1) interleaved at random positions
    npad = len(slots) // 9
    total = len(slots) + npad
    padpos = np.zeros(total, bool)
    padpos[rng.choice(total, npad, replace=False)] = True
    full = np.full(total, -1, np.int64)
    full[~padpos] = slots
    T = total
    g = torch.Generator(device=cuda).manual_seed(5)
    key = torch.randn(T, h, e, generator=g, device=cuda).to(torch.bfloat16)
    value = torch.randn(T, h, e, generator=g, device=cuda).to(torch.bfloat16)
    kc = torch.zeros(nb, h, page, e, dtype=torch.bfloat16, device=cuda)
    vc = torch.zeros_like(kc)
    reshape_and_cache(key, value, kc, vc, torch.from_numpy(full).to(cuda))
    kw = np.zeros((nb, h, page * e // 2), np.uint32)
    vw = np.zeros_like(kw)
    layout.store(kw, vw, row_words(key), row_words(value), full, page)
    np.testing.assert_array_equal(cache_words(kc), kw)
    np.testing.assert_array_equal(cache_words(vc), vw)
    prefix = lens
    cur = torch.tensor(prefix, dtype=torch.int32, device=cuda)
    tcuda = table.to(cuda)
    check_rows = [0, 31, 64, 127]
    for step in range(steps):
        q = torch.randn(n, 1, h, e, generator=g, device=cuda).to(torch.bfloat16)
        kn = torch.randn(n, 1, h, e, generator=g, device=cuda).to(torch.bfloat16)
        vn = torch.randn(n, 1, h, e, generator=g, device=cuda).to(torch.bfloat16)
        out = flash_attn_with_kvcache(q, kc, vc, k=kn, v=vn, cache_seqlens=cur, page_table=tcuda)
        s_np = layout.append_slots(cur.cpu().numpy(), table.numpy(), page)
        layout.store(kw, vw, row_words(kn[:, 0]), row_words(vn[:, 0]), s_np, page)
        cur = cur + 1
        # every step: the pages the step appended to, byte for byte
        blocks = np.unique(s_np[s_np >= 0] // page)
        bsel = torch.from_numpy(blocks).to(cuda)
        np.testing.assert_array_equal(cache_words(kc[bsel]), kw[blocks])
        np.testing.assert_array_equal(cache_words(vc[bsel]), vw[blocks])
        if step in (0, steps - 1):
            np.testing.assert_array_equal(cache_words(kc), kw)
            np.testing.assert_array_equal(cache_words(vc), vw)
            cl = cur.cpu().numpy()
            for s in check_rows:
                k, v = dense_kv(kc, vc, table[s], int(cl[s]), page)
                ref = attention(values(q[s:s + 1]), k[None], v[None], e ** -0.5)
                assert_close(out[s:s + 1], ref, torch.bfloat16, paged=True)
    assert torch.isfinite(out).all()
    K.module()  # the library stayed loaded and usable
