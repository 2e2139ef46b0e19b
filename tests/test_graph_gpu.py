"""The serving steps inside a HIP graph: decode, store, prompt append and prefill, as the
reference's engine use (examples/ops.py:19-31) would replay a captured step.  With
host checks off a valid call reads nothing on the host, synchronises nothing and
allocates only through torch (from the graph's pool while capturing), so it
captures as is.

Each test captures once, then replays several times with new inputs written into
the captured tensors. Before each replay an eager call runs on copies of the
caches, with synchronisations around the replay. The replay must match that eager
call bit for bit, in its output and in the caches it writes (bytewise, since the
caches keep NaN in slots no kernel may read). Rows past 2048 keys add the decode
workspace and its second kernel to the graph."""

import pytest
import torch

from cpu_attention import _kernel as K
from cpu_attention import flash_attn_func, flash_attn_with_kvcache, reshape_and_cache
from helpers import stage

pytestmark = pytest.mark.gpu
DTYPES = [torch.float32, torch.bfloat16]
# Appended tokens land inside allocated pages (no length is a multiple of 16); the
# last row walks 3004 keys, past one decode block's 2048.
LENS, H, D, PAGE = [30, 69, 1, 3003], 4, 128, 16


def same_bytes(a, b):
    return torch.equal(a.view(torch.uint8), b.view(torch.uint8))


def capture(fn):
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            fn()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = fn()
    return graph, out


@pytest.fixture
def no_host_checks():
    old = K.set_host_checks(False)
    yield
    K.set_host_checks(old)


@pytest.mark.parametrize("dtype", DTYPES)
def test_flash_attn_with_kvcache_append_replays(cuda, dtype, no_host_checks):
    q0, kc, vc, bt, _, _ = stage(LENS, H, D, PAGE, dtype, seed=31, device=cuda)
    b = len(LENS)
    lens = torch.tensor(LENS, dtype=torch.int32, device=cuda)
    sq, sk, sv = (torch.zeros(b, 1, H, D, dtype=dtype, device=cuda) for _ in range(3))
    graph, out = capture(lambda: flash_attn_with_kvcache(sq, kc, vc, k=sk, v=sv, cache_seqlens=lens,
                                                          page_table=bt))
    g = torch.Generator(device=cuda).manual_seed(5)
    for _ in range(4):
        for t in (sq, sk, sv):
            t.copy_(torch.randn(t.shape, generator=g, device=cuda).to(dtype))
        kr, vr = kc.clone(), vc.clone()
        ref = flash_attn_with_kvcache(sq.clone(), kr, vr, k=sk.clone(), v=sv.clone(), cache_seqlens=lens,
                                      page_table=bt)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.isfinite(out).all()
        assert same_bytes(out, ref)
        assert same_bytes(kc, kr) and same_bytes(vc, vr)


@pytest.mark.parametrize("dtype", DTYPES)
def test_large_batch_append_replays(cuda, dtype, no_host_checks):
    """Past 1024 (sequence, head) rows the one-token append is a separate scatter
    kernel before the decode: both dispatches inside the graph."""
    import random
    rng = random.Random(3)
    lens_host = [rng.randrange(1, 60) * 2 + 1 for _ in range(300)]  # odd: never a page edge
    q0, kc, vc, bt, _, _ = stage(lens_host, H, D, PAGE, dtype, seed=33, device=cuda)
    b = len(lens_host)
    assert b * H > 1024
    lens = torch.tensor(lens_host, dtype=torch.int32, device=cuda) - 1  # the append overwrites the last
    sq, sk, sv = (torch.zeros(b, 1, H, D, dtype=dtype, device=cuda) for _ in range(3))
    graph, out = capture(lambda: flash_attn_with_kvcache(sq, kc, vc, k=sk, v=sv, cache_seqlens=lens,
                                                          page_table=bt))
    g = torch.Generator(device=cuda).manual_seed(6)
    for _ in range(3):
        for t in (sq, sk, sv):
            t.copy_(torch.randn(t.shape, generator=g, device=cuda).to(dtype))
        kr, vr = kc.clone(), vc.clone()
        ref = flash_attn_with_kvcache(sq.clone(), kr, vr, k=sk.clone(), v=sv.clone(), cache_seqlens=lens,
                                      page_table=bt)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.isfinite(out).all()
        assert same_bytes(out, ref)
        assert same_bytes(kc, kr) and same_bytes(vc, vr)


@pytest.mark.parametrize("dtype", DTYPES)
def test_engine_step_with_slots_and_out_replays(cuda, dtype, no_host_checks):
    """The engine entry: store each new token at ``slots`` (one sequence skips with
    -1), lens is the post-store length, the caller owns ``out``."""
    q0, kc, vc, bt, _, _ = stage(LENS, H, D, PAGE, dtype, seed=32, device=cuda)
    b = len(LENS)
    pos = torch.tensor(LENS)
    slots = (bt.cpu()[torch.arange(b), pos // PAGE].long() * PAGE + pos % PAGE)
    slots[2] = -1
    slots = slots.to(cuda)
    post = torch.tensor([n + 1 for n in LENS], dtype=torch.int32, device=cuda)
    post[2] = LENS[2]
    sq, sk, sv = (torch.zeros(b, H, D, dtype=dtype, device=cuda) for _ in range(3))
    out = torch.empty_like(sq)
    mod, rt = K.module(), K.runtime()
    graph, got = capture(lambda: mod.decode(rt, sq, kc, vc, sk, sv, slots, post, bt, None, out))
    assert got is out
    g = torch.Generator(device=cuda).manual_seed(6)
    for _ in range(4):
        for t in (sq, sk, sv):
            t.copy_(torch.randn(t.shape, generator=g, device=cuda).to(dtype))
        kr, vr, ref = kc.clone(), vc.clone(), torch.empty_like(out)
        assert mod.decode(rt, sq.clone(), kr, vr, sk.clone(), sv.clone(), slots, post, bt, None, ref) is ref
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.isfinite(out).all()
        assert same_bytes(out, ref)
        assert same_bytes(kc, kr) and same_bytes(vc, vr)


@pytest.mark.parametrize("dtype", DTYPES)
def test_reshape_and_cache_replays(cuda, dtype, no_host_checks):
    """vLLM's store step: a token stride of a fused projection, one padding slot."""
    _, kc, vc, bt, _, _ = stage(LENS, H, D, PAGE, dtype, seed=33, device=cuda)
    pos = torch.tensor(LENS)
    slots = (bt.cpu()[torch.arange(len(LENS)), pos // PAGE].long() * PAGE + pos % PAGE)
    slots[1] = -1
    slots = slots.to(cuda)
    kv = torch.zeros(len(LENS), 3 * H * D, dtype=dtype, device=cuda)
    key, value = kv[:, :H * D].view(-1, H, D), kv[:, 2 * H * D:].view(-1, H, D)
    graph, _ = capture(lambda: reshape_and_cache(key, value, kc, vc, slots))
    g = torch.Generator(device=cuda).manual_seed(7)
    for _ in range(4):
        kv.copy_(torch.randn(kv.shape, generator=g, device=cuda).to(dtype))
        kr, vr = kc.clone(), vc.clone()
        reshape_and_cache(key.clone(), value.clone(), kr, vr, slots)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert same_bytes(kc, kr) and same_bytes(vc, vr)


@pytest.mark.parametrize("dtype", DTYPES)
def test_prompt_append_replays(cuda, dtype, no_host_checks):
    """A prompt stage: 5 new tokens per sequence appended and attended in one call."""
    lens = [20, 33, 3, 2001]
    q0, kc, vc, bt, _, _ = stage(lens, H, D, PAGE, dtype, seed=34, device=cuda)
    b = len(lens)
    cl = torch.tensor(lens, dtype=torch.int32, device=cuda)
    sq = torch.zeros(b, 1, H, D, dtype=dtype, device=cuda)
    sk, sv = (torch.zeros(b, 5, H, D, dtype=dtype, device=cuda) for _ in range(2))
    graph, out = capture(lambda: flash_attn_with_kvcache(sq, kc, vc, k=sk, v=sv, cache_seqlens=cl,
                                                          page_table=bt))
    g = torch.Generator(device=cuda).manual_seed(8)
    for _ in range(3):
        for t in (sq, sk, sv):
            t.copy_(torch.randn(t.shape, generator=g, device=cuda).to(dtype))
        kr, vr = kc.clone(), vc.clone()
        ref = flash_attn_with_kvcache(sq.clone(), kr, vr, k=sk.clone(), v=sv.clone(), cache_seqlens=cl,
                                      page_table=bt)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.isfinite(out).all()
        assert same_bytes(out, ref)
        assert same_bytes(kc, kr) and same_bytes(vc, vr)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("sq,sk", [(300, 300), (3, 3000), (1, 5000), (64, 3000)])
def test_flash_attn_func_replays(cuda, dtype, sq, sk):
    """Prefill: the tiled route, the few-rows route (per-head, and for one query
    row of 16 side-by-side heads the packed-heads kernel, both with split keys and
    the combine kernel) and the tiled route's split mode (64 rows over 3000 keys:
    11 splits and the combine kernel), whose split-K scratch is allocated inside
    the capture from the graph's own pool."""
    b, h, d = 2, (16 if sq == 1 else 4), 64
    q, k, v = (torch.zeros(b, n, h, d, dtype=dtype, device=cuda) for n in (sq, sk, sk))
    graph, out = capture(lambda: flash_attn_func(q, k, v, causal=True))
    g = torch.Generator(device=cuda).manual_seed(9)
    for i in range(3):
        for t in (q, k, v):
            t.copy_(torch.randn(t.shape, generator=g, device=cuda).to(dtype))
        ref = flash_attn_func(q.clone(), k.clone(), v.clone(), causal=True)
        if i == 1:
            # A larger eager call between replays (more scratch than the captured
            # one): the graph keeps its own scratch, so the replay is unaffected.
            big = torch.randn(b, sq, h, d, generator=g, device=cuda).to(dtype)
            bigk = torch.randn(b, 4 * sk, h, d, generator=g, device=cuda).to(dtype)
            flash_attn_func(big, bigk, bigk, causal=True)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.isfinite(out).all()
        assert same_bytes(out, ref)
