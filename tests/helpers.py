"""Shared helpers for the GPU parity tests: staging caches through the public API
the way the reference's tests do, and the float64 oracle on torch tensors."""

import numpy as np
import torch

from cpu_attention import flash_attn_with_kvcache
from oracle import layout
from oracle.attention import BF16, FP32, attention, check, gate

NAME = {torch.float32: FP32, torch.bfloat16: BF16}


def values(t):
    """Exact float64 values of a tensor (bf16 widens exactly)."""
    return t.detach().float().cpu().numpy().astype(np.float64)


def stage(lens, h, d, page, dtype, seed, device):
    """Caches holding ``lens[i]`` random tokens per sequence, staged through the API in
    two appends each (the reference's tests/test_kvcache.py:16-39).  Everything a
    kernel must not read is NaN: unused slots and pages, and the page-table
    padding (which points at a poisoned page)."""
    g = torch.Generator().manual_seed(seed)
    npages = [-(-n // page) for n in lens]
    total = sum(npages) + 1
    order = torch.randperm(total, generator=g).to(torch.int32)
    bt = torch.full((len(lens), max(npages) + 1), int(order[-1]), dtype=torch.int32)
    kc = torch.full((total, h, page, d), float("nan"), dtype=dtype, device=device)
    vc = kc.clone()
    q = torch.randn(len(lens), 1, h, d, generator=g).to(dtype).to(device)
    ks, vs, start = [], [], 0
    for i, n in enumerate(lens):
        bt[i, :npages[i]] = order[start:start + npages[i]]
        start += npages[i]
    btd = bt.to(device)
    for i, n in enumerate(lens):
        k, v = (torch.randn(1, n, h, d, generator=g).to(dtype).to(device) for _ in range(2))
        for a, z in ((0, n // 2), (n // 2, n)):
            if z > a:
                flash_attn_with_kvcache(q[i:i + 1], kc, vc, k=k[:, a:z], v=v[:, a:z],
                                        cache_seqlens=a, page_table=btd[i:i + 1])
        ks.append(k)
        vs.append(v)
    return q, kc, vc, btd, ks, vs


def reference(q, ks, vs, scale):
    """float64 decode reference: each sequence's row against its dense K/V."""
    return np.concatenate([attention(values(q[i:i + 1]), values(k), values(v), scale)
                           for i, (k, v) in enumerate(zip(ks, vs))])


def appended(ks, vs, kn, vn):
    return ([torch.cat([k, kn[i:i + 1]], 1) for i, k in enumerate(ks)],
            [torch.cat([v, vn[i:i + 1]], 1) for i, v in enumerate(vs)])


def assert_close(out, ref, dtype, paged):
    """The reference's gate and the MI355X build's gate."""
    got = values(out)
    assert np.all(np.isfinite(got)), "non-finite output"
    err, tol = check(got, ref, NAME[dtype], paged=paged)
    assert err <= tol, (err, tol)
    err, tol = gate(got, ref, NAME[dtype])
    assert err <= tol, (err, tol)


def cache_words(cache):
    """A cache tensor as numpy uint32 words [NB, H, P*W] (bytes, NaNs included)."""
    nb, h = cache.shape[:2]
    return cache.detach().contiguous().view(torch.int32).cpu().numpy().view(np.uint32).reshape(nb, h, -1) \
        if cache.dtype == torch.float32 else \
        cache.detach().contiguous().view(torch.int16).cpu().numpy().view(np.uint16).view(np.uint32).reshape(nb, h, -1)


def row_words(x):
    """key/value rows [T, H, E] as uint32 words [T, H, W]."""
    x = x.detach().contiguous()
    if x.dtype == torch.float32:
        return x.view(torch.int32).cpu().numpy().view(np.uint32)
    return x.view(torch.int16).cpu().numpy().view(np.uint16).view(np.uint32).reshape(*x.shape[:-1], -1)


__all__ = ["NAME", "values", "stage", "reference", "appended", "assert_close", "cache_words",
           "row_words", "layout", "attention"]
