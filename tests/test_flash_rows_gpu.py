"""flash_attn_func calls with few query rows (up to 4 in bf16; in fp32 up to 8, or
16 when batch x heads is 256 or more), which
take the split-K few-rows route, against the float64 oracle.  Covers every head
dim and dtype, key lengths at and past the chunk edges (one chunk, several, a
partial last one), single rows and row groups of 4 with a partial last group,
causal rows that see no key, strided q/k/v views, the boundary with the tiled
route, the cross shape of the BASELINE prefill config, and the workspace
protocol (the entry reports the bytes it needs; the API allocates them per call)."""

import numpy as np
import pytest
import torch

from cpu_attention import _kernel as K
from cpu_attention import flash_attn_func
from helpers import assert_close, attention, values

pytestmark = pytest.mark.gpu
DTYPES = [torch.float32, torch.bfloat16]


def run(b, sq, sk, h, d, dtype, causal, seed, device, scale=None):
    g = torch.Generator().manual_seed(seed)
    q, k, v = (torch.randn(b, n, h, d, generator=g).to(dtype).to(device) for n in (sq, sk, sk))
    out = flash_attn_func(q, k, v, softmax_scale=scale, causal=causal)
    assert out.shape == q.shape and out.dtype == dtype and out.is_contiguous()
    ref = attention(values(q), values(k), values(v), scale or d ** -0.5, causal)
    assert_close(out, ref, dtype, paged=False)
    return out


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("d", [32, 64, 128])
@pytest.mark.parametrize("sq", [1, 2, 3, 4, 5, 8, 16])
@pytest.mark.parametrize("sk", [1, 31, 32, 33, 128, 129, 300, 1100])
@pytest.mark.parametrize("causal", [True, False])
def test_few_rows_shapes(cuda, dtype, d, sq, sk, causal):
    run(2, sq, sk, 3, d, dtype, causal, seed=sq * 10000 + sk * 10 + d, device=cuda)


@pytest.mark.parametrize("dtype,sq,h", [(torch.bfloat16, 4, 4), (torch.bfloat16, 5, 4),
                                        (torch.float32, 8, 4), (torch.float32, 9, 4),
                                        (torch.float32, 12, 128), (torch.float32, 13, 128), (torch.float32, 16, 128),
                                        (torch.float32, 17, 128)])
def test_route_boundary(cuda, dtype, sq, h):
    """The last row count of the few-rows route and the first of the tiled one
    both agree with the oracle: bf16 4 | 5; fp32 8 | 9 with 8 (batch, head) pairs,
    and 16 | 17 with 256 pairs (12 rows: three row groups of 4; 13 and 16 rows: row
    groups of 8, the last one partial or full)."""
    run(2, sq, 700, h, 64, dtype, True, seed=sq, device=cuda)


@pytest.mark.parametrize("d", [32, 64, 128])
@pytest.mark.parametrize("sq,sk", [(13, 100), (16, 2000), (14, 4096)])
@pytest.mark.parametrize("causal", [True, False])
def test_fp32_row_groups_of_eight(cuda, d, sq, sk, causal):
    """fp32 calls of 13 to 16 rows with 256 (batch, head) pairs run 8 rows per wave
    (two waves read each key instead of four): partial and full groups, causal rows
    that see fewer keys than the group's widest, short and long key ranges."""
    print(f"fp32 row groups of eight sq={sq} sk={sk} d={d} causal={causal}", flush=True)
    run(4, sq, sk, 64, d, torch.float32, causal, seed=sq * 100 + d, device=cuda)


@pytest.mark.parametrize("dtype", DTYPES)
def test_causal_rows_without_keys(cuda, dtype):
    """seq_q > seq_k: the first seq_q - seq_k rows see no key and are exactly 0."""
    out = run(1, 16, 5, 2, 64, dtype, True, seed=3, device=cuda)
    assert torch.count_nonzero(out[:, :11]) == 0


@pytest.mark.parametrize("dtype", DTYPES)
def test_strided_views(cuda, dtype):
    """q/k/v as chunks of a fused projection (token stride 3*H*E), with a batch
    stride that is not a multiple of the token stride."""
    b, sq, sk, h, d = 3, 3, 500, 4, 32
    g = torch.Generator().manual_seed(5)
    kv = torch.randn(b, sk + 7, 3 * h * d, generator=g).to(dtype).to(cuda)[:, :sk]
    k, v = (kv[..., i * h * d:(i + 1) * h * d].view(b, sk, h, d) for i in (0, 2))
    q = torch.randn(b, sq, h, d, generator=g).to(dtype).to(cuda)
    out = flash_attn_func(q, k, v, causal=False)
    assert_close(out, attention(values(q), values(k), values(v), d ** -0.5), dtype, paged=False)


def heads_per_load(d, dtype):
    """Heads one wave load instruction covers on the single-row route for packed
    heads (64 lanes of 16 bytes over rows of d elements; csrc/ca_rows.hip)."""
    return 64 // (d * dtype.itemsize // 16)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("d", [32, 64, 128])
@pytest.mark.parametrize("sk", [1, 5, 64, 300, 1024, 1025, 2049, 8191])
def test_single_row_packed_heads(cuda, dtype, d, sk):
    """One query row with the heads side by side (head stride d) and a head count
    that is a multiple of the heads per load: the route that reads each key's
    heads as one run, with the keys split over blocks and merged by the combine
    kernel; also with k/v as chunks of a fused projection (still packed heads)."""
    h = 2 * heads_per_load(d, dtype)
    run(3, 1, sk, h, d, dtype, False, seed=sk + d, device=cuda)
    g = torch.Generator().manual_seed(sk)
    kv = torch.randn(2, sk, 2 * h * d, generator=g).to(dtype).to(cuda)
    k, v = (kv[..., i * h * d:(i + 1) * h * d].view(2, sk, h, d) for i in (0, 1))
    q = torch.randn(2, 1, h, d, generator=g).to(dtype).to(cuda)
    out = flash_attn_func(q, k, v, causal=True)
    assert_close(out, attention(values(q), values(k), values(v), d ** -0.5, True), dtype, paged=False)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("d", [32, 128])
@pytest.mark.parametrize("packed", [True, False])
def test_most_splits(cuda, dtype, d, packed):
    """One (batch, head group) over 40000 keys: its keys split over 64 blocks, the
    most there are, so the combine gives every lane of its wave a split (weights
    read across the lanes).  Packed: one group of heads per load on the
    packed-heads route; unpacked: one head on the per-head route, and 3 rows in
    one group."""
    sk = 40000
    h = heads_per_load(d, dtype) if packed else 1
    lib = K.load_library()
    if packed:
        need = lib.ca_flash_workspace_bytes(1, 1, sk, h, d, K.DTYPES[dtype])
        assert need == h * 64 * (d + 2) * 4  # 64 splits
        run(1, 1, sk, h, d, dtype, False, seed=d + 1, device=cuda)
    else:
        need = lib.ca_flash_workspace_bytes(1, 3, sk, 1, d, K.DTYPES[dtype])
        assert need == 3 * 64 * (d + 2) * 4
        run(1, 3, sk, 1, d, dtype, False, seed=d + 2, device=cuda)
        run(1, 1, sk, 1, d, dtype, True, seed=d + 3, device=cuda)


@pytest.mark.parametrize("dtype", DTYPES)
def test_single_row_unpacked_heads(cuda, dtype):
    """One query row whose k/v heads are not side by side (head stride 2d, a
    strided view) takes the per-head route and agrees as well."""
    d, sk = 64, 1000
    h = heads_per_load(d, dtype)
    g = torch.Generator().manual_seed(4)
    kv = torch.randn(2, sk, h, 2 * d, generator=g).to(dtype).to(cuda)
    k, v = kv[..., :d], kv[..., d:]
    assert k.stride(2) == 2 * d
    q = torch.randn(2, 1, h, d, generator=g).to(dtype).to(cuda)
    out = flash_attn_func(q, k, v)
    assert_close(out, attention(values(q), values(k), values(v), d ** -0.5), dtype, paged=False)


def test_scale_and_large_logits(cuda):
    """A large scale (logits spread over many chunks' maxima) in fp32."""
    run(2, 4, 2000, 2, 128, torch.float32, False, seed=9, device=cuda, scale=0.5)


def test_cfg4_cross_shape_rows(cuda):
    """BASELINE cfg4's cross shape: N=8 L=1 S=2048 E=32 H=32, non-causal, bf16."""
    run(8, 1, 2048, 32, 32, torch.bfloat16, False, seed=12, device=cuda)


def test_few_rows_calls_on_two_streams(cuda):
    """Split-K calls queued on two streams at once, each with its own scratch: the
    partials of one never land in the other's (a scratch shared per thread
    would race here)."""
    b, sq, sk, h, d = 2, 2, 3000, 8, 64
    g = torch.Generator().manual_seed(21)
    cases = [tuple(torch.randn(b, n, h, d, generator=g).bfloat16().to(cuda) for n in (sq, sk, sk))
             for _ in range(2)]
    streams = [torch.cuda.Stream(device=cuda) for _ in range(2)]
    torch.cuda.synchronize()
    outs = []
    for _ in range(4):
        for (q, k, v), st in zip(cases, streams):
            with torch.cuda.stream(st):
                outs.append(flash_attn_func(q, k, v, causal=False))
    torch.cuda.synchronize()
    for i, out in enumerate(outs):
        q, k, v = cases[i % 2]
        assert_close(out, attention(values(q), values(k), values(v), d ** -0.5), torch.bfloat16, paged=False)


def test_engine_workspace_per_stream(cuda):
    """``K.workspace()`` (for callers of the module entry) keeps one buffer per
    stream and grows it only upward."""
    a = K.workspace(1000)
    assert a[1] >= 1000 and K.workspace() == a
    st = torch.cuda.Stream(device=cuda)
    with torch.cuda.stream(st):
        assert K.workspace() == (0, 0)
        b = K.workspace(10)
        assert b[0] != a[0]
    assert K.workspace(10) == a
    # releasing the side stream's buffers leaves the current stream's alone
    with torch.cuda.stream(st):
        assert K.release_workspace() == 1
        assert K.workspace() == (0, 0)
    assert K.workspace() == a
    K.workspace(4 * a[1])  # outgrown: both buffers stay until released
    assert K.release_workspace(all_streams=True) == 2
    assert K.workspace() == (0, 0)


def test_native_entry_reports_the_workspace_it_needs(cuda):
    """The module entry returns the bytes it needs (an int) when the workspace is short."""
    mod, rt = K.module(), K.runtime()
    q = torch.randn(1, 1, 4, 64, device=cuda)
    k = torch.randn(1, 4000, 4, 64, device=cuda)
    need = mod.flash(rt, q, k, k, None, False, 0, 0)
    assert type(need) is int and need > 0
    ws = torch.empty(need, dtype=torch.uint8, device=cuda)
    out = mod.flash(rt, q, k, k, None, False, ws.data_ptr(), need)
    ref = attention(values(q), values(k), values(k), 64 ** -0.5)
    assert np.abs(values(out) - ref).max() <= 1e-5
