"""flash_attn_func on the GPU against the float64 oracle.  Mirrors the reference's
tests/test_flash.py case for case (shape grid with tile edges and unequal lengths,
batch and scale, fused-qkv strides, fuzz, repeated calls), then adds the
BASELINE prefill shapes, rows with no visible key, and layouts that need a copy."""

import random

import numpy as np
import pytest
import torch

from cpu_attention import flash_attn_func
from helpers import assert_close, attention, values
from route_cases import SEEDS as ROUTE_SEEDS, route_case

pytestmark = pytest.mark.gpu
DTYPES = [torch.float32, torch.bfloat16]
# (seq_q, seq_k): tile edges (16/64/128 rows), single rows, unequal lengths both ways.
LENGTHS = [(1, 1), (17, 17), (64, 64), (129, 129), (1, 300), (100, 37), (37, 100), (257, 513)]


def run(b, sq, sk, h, d, dtype, causal, seed, device, scale=None):
    g = torch.Generator().manual_seed(seed)
    q, k, v = (torch.randn(b, n, h, d, generator=g).to(dtype).to(device) for n in (sq, sk, sk))
    out = flash_attn_func(q, k, v, softmax_scale=scale, causal=causal)
    assert out.shape == q.shape and out.dtype == dtype and out.is_contiguous()
    ref = attention(values(q), values(k), values(v), scale or d ** -0.5, causal)
    assert_close(out, ref, dtype, paged=False)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("d", [32, 64, 128])
@pytest.mark.parametrize("sq,sk", LENGTHS)
@pytest.mark.parametrize("h", [1, 8])
@pytest.mark.parametrize("causal", [True, False])
def test_shapes(cuda, dtype, d, sq, sk, h, causal):
    run(1, sq, sk, h, d, dtype, causal, seed=sq * 1000 + sk, device=cuda)


@pytest.mark.parametrize("dtype", DTYPES)
def test_batch_and_scale(cuda, dtype):
    run(3, 70, 150, 8, 64, dtype, True, seed=1, device=cuda, scale=0.07)


@pytest.mark.parametrize("dtype", DTYPES)
def test_fused_qkv_strides(cuda, dtype):
    """q/k/v as chunks of one [b, s, 3*h*d] projection (no copy is needed)."""
    b, s, h, d = 2, 200, 4, 64
    qkv = torch.randn(b, s, 3 * h * d).to(dtype).to(cuda)
    q, k, v = (qkv[..., i * h * d:(i + 1) * h * d].view(b, s, h, d) for i in range(3))
    out = flash_attn_func(q, k, v, causal=True)
    assert_close(out, attention(values(q), values(k), values(v), d ** -0.5, True), dtype, paged=False)


@pytest.mark.parametrize("seed", range(40))
def test_fuzz(cuda, seed):
    r = random.Random(seed)
    run(r.randint(1, 3), r.randint(1, 900), r.randint(1, 900), r.choice([1, 4, 12]),
        r.choice([32, 64, 128]), r.choice(DTYPES), r.random() < 0.5, seed, cuda)


@pytest.mark.parametrize("seed", range(ROUTE_SEEDS))
def test_route_sweep(cuda, seed):
    """Seeded shapes weighted toward the route boundaries (short keys either side of
    256, few query blocks over long keys, a few query rows; route_cases), in three
    layouts.  Sampled rows of up to 12 (batch, head) pairs are checked against the
    float64 oracle over exactly the keys each row sees (bottom-right causal; a row
    that sees none is 0).  The CPU address check replays the same shapes."""
    b, sq, sk, h, d, dt, causal, layout = route_case(seed)
    dtype = torch.bfloat16 if dt == "bf16" else torch.float32
    print(f"route sweep {seed}: b={b} sq={sq} sk={sk} h={h} d={d} {dt} causal={causal} {layout}", flush=True)
    g = torch.Generator(device=cuda).manual_seed(seed)
    if layout == "fused":
        qkv = torch.randn(b, sq, 3 * h * d, generator=g, device=cuda).to(dtype)
        q, k, v = (qkv[..., i * h * d:(i + 1) * h * d].view(b, sq, h, d) for i in range(3))
    elif layout == "bhse":
        q, k, v = (torch.randn(b, h, n, d, generator=g, device=cuda).to(dtype).transpose(1, 2) for n in (sq, sk, sk))
    else:
        q, k, v = (torch.randn(b, n, h, d, generator=g, device=cuda).to(dtype) for n in (sq, sk, sk))
    out = flash_attn_func(q, k, v, causal=causal)
    r = random.Random(seed)
    rows = list(range(sq)) if sq * sk <= 300000 else sorted({0, sq - 1, *(r.randrange(sq) for _ in range(24))})
    pairs = [(bi, hi) for bi in range(b) for hi in range(h)]
    if len(pairs) > 12:
        pairs = r.sample(pairs, 12)
    for bi, hi in pairs:
        qv, kv, vv, ov = (values(t[bi:bi + 1, :, hi:hi + 1]) for t in (q, k, v, out))
        ref = []
        for i in rows:
            ke = min(sk, max(0, i + 1 + sk - sq)) if causal else sk
            ref.append(attention(qv[:, i:i + 1], kv[:, :ke], vv[:, :ke], d ** -0.5)[0, 0, 0] if ke else np.zeros(d))
        assert_close(torch.from_numpy(ov[0, rows, 0]), np.stack(ref), dtype, paged=False)


def test_repeated_calls_follow_changes(cuda):
    """The call plan must follow every change of scale, causal and shape."""
    for scale, causal, s in ((0.05, True, 64), (0.125, False, 64), (0.05, False, 65)):
        run(1, s, s, 4, 64, torch.float32, causal, seed=s, device=cuda, scale=scale)


@pytest.mark.parametrize("d", [32, 64, 128])
def test_waves_without_rows_leave_tiles_alone(cuda, d):
    """Causal calls with far fewer keys than queries: in a block, waves whose rows
    see no key only issue their share of the tile loads and wait at the barriers
    while the others read the tiles.  A load of theirs that refilled a buffer
    still being read (the pass's first K tile, a V tile read before its barrier)
    corrupted a few rows now and then; repeated calls must all hold."""
    for rep in range(6):
        run(2, 850, 86, 1, d, torch.bfloat16, True, seed=23 + rep, device=cuda)
        run(1, 700, 70, 4, d, torch.bfloat16, True, seed=7 + rep, device=cuda)


@pytest.mark.parametrize("dtype", DTYPES)
def test_rows_without_keys_are_zero(cuda, dtype):
    """Causal with seq_q > seq_k: the first seq_q - seq_k rows see no key and are 0."""
    g = torch.Generator().manual_seed(2)
    q = torch.randn(2, 300, 4, 64, generator=g).to(dtype).to(cuda)
    k = torch.randn(2, 90, 4, 64, generator=g).to(dtype).to(cuda)
    out = flash_attn_func(q, k, k, causal=True)
    assert torch.count_nonzero(out[:, :210]) == 0
    assert_close(out, attention(values(q), values(k), values(k), 64 ** -0.5, True), dtype, paged=False)


@pytest.mark.parametrize("dtype", DTYPES)
def test_layouts_needing_a_copy(cuda, dtype):
    """A head dim that is not contiguous, and a 16-byte-misaligned view, are copied
    by the Python layer and still computed correctly."""
    g = torch.Generator().manual_seed(3)
    base = torch.randn(1, 50, 4, 130, generator=g).to(dtype).to(cuda)
    q = base[..., 1:65]  # misaligned start, token/head strides not 16-byte multiples
    k = torch.randn(1, 64, 50, 4, generator=g).to(dtype).to(cuda).permute(0, 2, 3, 1)  # dim stride != 1
    v = torch.randn(1, 50, 4, 64, generator=g).to(dtype).to(cuda)
    out = flash_attn_func(q, k, v, causal=False)
    assert_close(out, attention(values(q), values(k), values(v), 64 ** -0.5), dtype, paged=False)


@pytest.mark.parametrize("causal", [True, False])
def test_north_star_tolerance_fp32(cuda, causal):
    """fp32 within 1e-5 relative of float64 (the north-star gate), longer rows."""
    run(1, 1000, 1000, 2, 128, torch.float32, causal, seed=5, device=cuda)


def test_cfg1_prefill_bf16(cuda):
    """BASELINE cfg1: N=1 L=S=128 H=16 E=64 causal bottom-right, bf16."""
    run(1, 128, 128, 16, 64, torch.bfloat16, True, seed=0, device=cuda)


def test_cfg4_cross_shape(cuda):
    """BASELINE cfg4 (its cross shape): N=8 L=1 S=2048 E=32 H=32, non-causal, bf16."""
    run(8, 1, 2048, 32, 32, torch.bfloat16, False, seed=8, device=cuda)


def test_cfg4_prefill_full_size_sampled(cuda):
    """BASELINE cfg4: N=4 L=S=4096 H=32 E=128 causal bf16, q/k/v strided chunks of a
    fused [N*L, 3*H*E] projection.  The whole output is computed; the float64 oracle
    checks every one of the 128 (batch, head) pairs, on one row of each 256-row
    query block (a different offset per pair and block, so both passes of every
    causal pair, every wave's rows and every block of the XCD schedule are seen)
    and on the first and last rows, plus tile and block edges of a few pairs."""
    N, L, H, E = 4, 4096, 32, 128
    g = torch.Generator(device=cuda).manual_seed(4)
    qkv = torch.randn(N * L, 3 * H * E, generator=g, device=cuda).to(torch.bfloat16)
    q, k, v = (qkv[:, i * H * E:(i + 1) * H * E].view(N, L, H, E) for i in range(3))
    out = flash_attn_func(q, k, v, causal=True)
    assert torch.isfinite(out).all()
    # Each row's reference is the oracle over exactly the keys it sees (j <= i at
    # L == S), under the reference's gate and the north star's.
    edges = [1, 63, 64, 255, 256, 2047, 2048, 3839, 3840, 4094]
    for b in range(N):
        for h in range(H):
            rows = [0, L - 1] + [256 * j + (37 * j + 11 * b + 5 * h + 3) % 256 for j in range(L // 256)]
            if (b * H + h) % 29 == 0:
                rows += edges
            rows = sorted(set(rows))
            kb, vb = values(k[b:b + 1, :, h:h + 1]), values(v[b:b + 1, :, h:h + 1])
            qb = values(q[b:b + 1, :, h:h + 1])
            got = values(out[b, rows, h])
            ref = np.stack([attention(qb[:, i:i + 1], kb[:, :i + 1], vb[:, :i + 1], E ** -0.5)[0, 0, 0]
                            for i in rows])
            assert_close(torch.from_numpy(got), ref, torch.bfloat16, paged=False)


@pytest.mark.parametrize("d", [32, 64, 128])
@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("gap", [40, 100, 180])
def test_logits_outgrowing_the_first_tile(cuda, d, causal, gap):
    """Keys far past the first 64 whose logits exceed every logit of the first key
    tile by about `gap` log2 units.  The bf16 kernel's fast walk fixes each row's
    max 64 units above the first tile's, so p reaches about 2^(gap - 64): up to a
    tile sum of 2^64 (gaps up to ~123) it carries on (the values are exact, only
    large), past that those rows are recomputed with a running max (some waves of a
    block take that path, others do not; at d = 32 the gap spreads widely over the
    rows, and some p overflow to inf before their wave is redone)."""
    g = torch.Generator().manual_seed(11)
    b, sq, sk, h = 2, 300, 700, 2
    q = (torch.randn(b, sq, h, d, generator=g) + 1.0).bfloat16()
    k = torch.randn(b, sk, h, d, generator=g)
    # q ~ N(1, 1): a key of constant `big` has a scaled logit near big * sqrt(d) *
    # log2(e) in log2 units, the others stay within a few units of 0
    big = (gap + 4) / (1.4427 * d ** 0.5)
    k[:, 200] = big
    k[:, 650] = big - 0.5
    k = k.bfloat16()
    v = torch.randn(b, sk, h, d, generator=g).bfloat16()
    q, k, v = q.to(cuda), k.to(cuda), v.to(cuda)
    out = flash_attn_func(q, k, v, causal=causal)
    ref = attention(values(q), values(k), values(v), d ** -0.5, causal)
    assert_close(out, ref, torch.bfloat16, paged=False)


@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("bad_pass", [0, 1])
def test_safe_pass_for_one_pass_of_a_causal_pair(cuda, d, bad_pass):
    """A causal call of two 256-row query blocks runs as one pair in one bf16 block:
    pass 0 (rows 256-511), then pass 1 (rows 0-255).  Only one of the two passes
    holds rows whose logits outgrow the fast walk's fixed max; the block redoes
    exactly those after both passes and keeps the other pass's fast results."""
    g = torch.Generator().manual_seed(12 + bad_pass)
    b, L, h = 1, 512, 130  # 260 query blocks: paired
    q = torch.randn(b, L, h, d, generator=g) * 0.5 + 1.0
    k = torch.randn(b, L, h, d, generator=g) * 0.5
    # a key whose logits sit about 180 log2 units above the first tile's max (past
    # the ~123 that the fast walk's fixed max and 2^64 headroom serve)
    big = 184 / (1.4427 * d ** 0.5)
    if bad_pass == 0:
        k[:, 400] = big  # seen only by rows >= 400 (pass 0)
    else:
        k[:, 200] = big  # seen by every row >= 200: rows of pass 0 get q < 0 for it
        q[:, 256:] = -q[:, 256:]
    q, k = q.bfloat16().to(cuda), k.bfloat16().to(cuda)
    v = torch.randn(b, L, h, d, generator=g).bfloat16().to(cuda)
    out = flash_attn_func(q, k, v, causal=True)
    for hh in (0, h - 1):
        sel = slice(hh, hh + 1)
        ref = attention(values(q[:, :, sel]), values(k[:, :, sel]), values(v[:, :, sel]), d ** -0.5, True)
        assert_close(out[:, :, sel], ref, torch.bfloat16, paged=False)


@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("causal,sq,h", [(True, 1536, 2), (False, 600, 2), (True, 1536, 44), (False, 600, 86)])
def test_every_wave_of_a_block_failing_the_walk(cuda, d, causal, sq, h):
    """Key 100 sits about 180 log2 units above every row's first-tile max (the fast
    walk serves ~123), so every wave whose rows see it fails the walk's headroom
    from tile 1 on, and
    whole blocks redo their rows in the safe pass.  Causal, 1536 rows: the pair
    (rows 1280-1535, rows 0-255) fails all of its first pass and part of its second
    (whose first wave never sees key 100).  Non-causal, 600 rows over 1536 keys:
    every full block fails; the last block's waves past row 599 do not.  With 2
    heads the query blocks are few, so their keys are split over blocks (the safe
    pass writes partials); with 44 or 86 heads they fill the chip (pairs when
    causal, one block per query block otherwise)."""
    g = torch.Generator().manual_seed(13)
    b = 1
    sk = 1536
    q = torch.randn(b, sq, h, d, generator=g) * 0.5 + 1.0
    k = torch.randn(b, sk, h, d, generator=g) * 0.5
    k[:, 100] = 184 / (1.4427 * d ** 0.5)
    q, k = q.bfloat16().to(cuda), k.bfloat16().to(cuda)
    v = torch.randn(b, sk, h, d, generator=g).bfloat16().to(cuda)
    out = flash_attn_func(q, k, v, causal=causal)
    for hh in (0, h - 1):
        sel = slice(hh, hh + 1)
        ref = attention(values(q[:, :, sel]), values(k[:, :, sel]), values(v[:, :, sel]), d ** -0.5, causal)
        assert_close(out[:, :, sel], ref, torch.bfloat16, paged=False)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("b,sq,sk,h", [(1, 600, 600, 130), (1, 400, 400, 8), (1, 2048, 2048, 32),
                                       (2, 700, 1200, 48), (1, 2048, 4096, 32), (1, 1024, 1024, 16),
                                       (1, 2048, 2048, 4), (1, 1500, 1500, 10), (1, 512, 512, 16),
                                       (1, 4096, 4096, 4), (1, 1500, 1500, 20), (1, 4096, 4096, 8)])
def test_causal_block_schedules(cuda, d, b, sq, sk, h, dtype):
    """The causal block schedules, each checked on a few heads: query-block pairs
    (qb, nqb-1-qb) in one block when unpaired blocks would leave the chip
    unevenly loaded, else one block per query block.  bf16 (256 rows per query
    block) pairs past 256: 1 x 130 x 3 = 390 (two pairs and one lone block per
    head) and 2 x 48 x 3 = 288 (more keys than rows) pair; 16 blocks over 400 keys
    (too few keys to split) and 256 at L = 2048 do not.  fp32 (128 rows) pairs
    from 1024, or from 512 with fewer than twice as many keys as rows: 650, 576
    and 512 at L = S = 2048 pair (odd and even counts per head); 32, and 512 over
    4096 keys, do not.  64 bf16 query blocks at L = S = 1024 run unsplit (causal
    triangle); the same call in fp32 (128 query blocks) splits its keys.  Fewer
    bf16 query blocks over at least 1024 keys split (32 at L = S = 2048: 8 splits;
    60 at L = S = 1500: 4), over 512 keys they do not; 64 to 127 split over 2048
    keys or more (64 at L = S = 4096: 4 splits), not below (120 at L = S = 1500),
    causal or not; 128 split in two over 4096 keys or more."""
    g = torch.Generator().manual_seed(40 + h)
    q = torch.randn(b, sq, h, d, generator=g).to(dtype).to(cuda)
    k, v = (torch.randn(b, sk, h, d, generator=g).to(dtype).to(cuda) for _ in range(2))
    out = flash_attn_func(q, k, v, causal=True)
    for hh in sorted({0, h // 2, h - 1}):
        sel = slice(hh, hh + 1)
        ref = attention(values(q[:, :, sel]), values(k[:, :, sel]), values(v[:, :, sel]), d ** -0.5, True)
        assert_close(out[:, :, sel], ref, dtype, paged=False)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_causal_pairs_with_rows_without_keys(cuda, dtype):
    """Causal pairs whose low query blocks see no key: 2304 rows over 1024 keys, 32
    heads (288 bf16 / 576 fp32 query blocks, both paired).  Rows below 1280 are
    exactly 0, written by the passes that have no key tile."""
    g = torch.Generator().manual_seed(50)
    b, sq, sk, h, d = 1, 2304, 1024, 32, 64
    q = torch.randn(b, sq, h, d, generator=g).to(dtype).to(cuda)
    k, v = (torch.randn(b, sk, h, d, generator=g).to(dtype).to(cuda) for _ in range(2))
    out = flash_attn_func(q, k, v, causal=True)
    assert torch.count_nonzero(out[:, :sq - sk]) == 0
    for hh in (0, 17, 31):
        sel = slice(hh, hh + 1)
        ref = attention(values(q[:, :, sel]), values(k[:, :, sel]), values(v[:, :, sel]), d ** -0.5, True)
        assert_close(out[:, :, sel], ref, dtype, paged=False)


# Calls whose query blocks leave most CUs idle split each query block's keys over
# several blocks (split mode of the tiled kernels): (batch, seq_q, seq_k, heads).
SPLIT_SHAPES = [(1, 64, 4096, 32), (1, 17, 2100, 8), (2, 300, 1500, 4), (1, 600, 4000, 3)]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("d", [32, 64, 128])
@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("shape", SPLIT_SHAPES)
def test_split_keys(cuda, d, causal, shape, dtype):
    """Few query rows over long key ranges, so the keys of each query block are
    split over several blocks and the row partials merged by the combine kernel:
    unequal lengths, partial last tiles and query blocks, causal ranges that end
    inside a split and splits past a query block's last key."""
    b, sq, sk, h = shape
    run(b, sq, sk, h, d, dtype, causal, 31 + sq, cuda)


@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("b,sq,sk,h", [(2, 600, 600, 8), (1, 512, 512, 8), (1, 768, 768, 4), (1, 1000, 1000, 2)])
def test_short_key_split_rule(cuda, d, b, sq, sk, h):
    """bf16 non-causal calls under 1024 keys (fewer than twice as many keys as
    rows): from 16 query blocks unsplit (48 and 16 here), below it their keys split
    over blocks (12 and 8)."""
    print(f"short-key split rule b={b} sq={sq} sk={sk} h={h} d={d}", flush=True)
    run(b, sq, sk, h, d, torch.bfloat16, False, 61 + sq, cuda)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_split_keys_rows_without_keys(cuda, dtype):
    """Causal with more query rows than keys: the first rows see no key (exactly
    0).  fp32 splits the keys over blocks (every split of those rows is empty);
    bf16 causal calls with fewer than twice as many keys as rows do not split
    below 1024 keys."""
    g = torch.Generator().manual_seed(32)
    q = torch.randn(1, 700, 4, 64, generator=g).to(dtype).to(cuda)
    k, v = (torch.randn(1, 600, 4, 64, generator=g).to(dtype).to(cuda) for _ in range(2))
    out = flash_attn_func(q, k, v, causal=True)
    assert torch.count_nonzero(out[:, :100]) == 0
    ref = attention(values(q), values(k), values(v), 64 ** -0.5, True)
    assert_close(out, ref, dtype, paged=False)


@pytest.mark.parametrize("d", [64, 128])
def test_split_keys_safe_pass(cuda, d):
    """A key about 180 log2 units above its split's first tile (the fast walk
    serves ~123): the waves of the split that holds it redo their rows in the safe
    pass, which writes partials for the combine like the fast walk."""
    g = torch.Generator().manual_seed(33)
    b, sq, sk, h = 1, 64, 4096, 8
    q = torch.randn(b, sq, h, d, generator=g) * 0.5 + 1.0
    k = torch.randn(b, sk, h, d, generator=g) * 0.5
    k[:, 2100] = 184 / (1.4427 * d ** 0.5)
    q, k = q.bfloat16().to(cuda), k.bfloat16().to(cuda)
    v = torch.randn(b, sk, h, d, generator=g).bfloat16().to(cuda)
    for causal in (False, True):
        out = flash_attn_func(q, k, v, causal=causal)
        ref = attention(values(q), values(k), values(v), d ** -0.5, causal)
        assert_close(out, ref, torch.bfloat16, paged=False)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_split_keys_module_asks_for_workspace(cuda, dtype):
    """The native module's flash returns the workspace bytes a split call needs when
    it gets less (the reference's grow-and-retry, flash_attn_interface.py:186-193)."""
    from cpu_attention import _kernel as K
    mod = K.module()
    q = torch.randn(1, 64, 32, 128, device=cuda).to(dtype)
    k = torch.randn(1, 4096, 32, 128, device=cuda).to(dtype)
    need = mod.flash(K.runtime(), q, k, k, None, False, None, 0)
    splits = 8 if dtype == torch.bfloat16 else 16  # 32 query blocks against 256 / 512 target blocks
    assert isinstance(need, int) and need == 32 * 64 * splits * 130 * 4
    ws = torch.empty(need, dtype=torch.uint8, device=cuda)
    out = mod.flash(K.runtime(), q, k, k, None, False, ws.data_ptr(), need)
    ref = attention(values(q), values(k), values(k), 128 ** -0.5, False)
    assert_close(out, ref, dtype, paged=False)


def strided(x, layout):
    """The same values as a view with the given layout: a chunk of a fused
    [b, s, 3 * h * d] projection, or a head-major [b, h, s, d] tensor viewed as
    [b, s, h, d]."""
    b, s, h, d = x.shape
    if layout == "fused":
        buf = torch.zeros(b, s, 3 * h * d, dtype=x.dtype, device=x.device)
        buf[..., h * d:2 * h * d] = x.reshape(b, s, h * d)
        return buf[..., h * d:2 * h * d].view(b, s, h, d)
    if layout == "bhse":
        return x.permute(0, 2, 1, 3).contiguous().permute(0, 2, 1, 3)
    return x


@pytest.mark.parametrize("d", [32, 64, 128])
@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("layout", ["contiguous", "fused", "bhse"])
@pytest.mark.parametrize("b,sq,sk,h", [(1, 128, 128, 16), (2, 5, 128, 3), (1, 200, 37, 4), (3, 33, 97, 2),
                                       (1, 64, 1, 8), (2, 31, 64, 5), (1, 96, 32, 1), (1, 256, 256, 4),
                                       (2, 129, 129, 3), (1, 40, 193, 2), (1, 250, 225, 2)])
def test_short_key_ranges(cuda, d, causal, layout, b, sq, sk, h):
    """bf16 calls of at most 256 keys (the short-key route: one wave per 32 query
    rows, every key in registers): partial 32-key blocks, a single key, more rows
    than keys (causal rows that see no key are 0), more keys than rows, partial
    32-row blocks, and q/k/v read in place from fused or head-major views."""
    g = torch.Generator().manual_seed(sq * 131 + sk)
    q, k, v = (strided(torch.randn(b, n, h, d, generator=g).bfloat16().to(cuda), layout) for n in (sq, sk, sk))
    out = flash_attn_func(q, k, v, causal=causal)
    ref = attention(values(q), values(k), values(v), d ** -0.5, causal)
    assert_close(out, ref, torch.bfloat16, paged=False)
    if causal and sq > sk:
        assert torch.count_nonzero(out[:, :sq - sk]) == 0


@pytest.mark.parametrize("b,sq,sk,h,d", [(8, 128, 128, 32, 64), (8, 129, 128, 32, 64), (2, 32, 256, 4, 64),
                                         (2, 32, 257, 4, 64), (3, 256, 256, 32, 64), (4, 256, 256, 32, 64),
                                         (4, 256, 192, 32, 64), (8, 256, 256, 16, 32), (2, 256, 256, 32, 128),
                                         (3, 256, 256, 32, 128), (3, 160, 160, 32, 128), (4, 160, 160, 32, 128)])
def test_short_key_route_edges(cuda, b, sq, sk, h, d):
    """Either side of the short-key route's limits: 8 x 32 x 4 = 1024 row blocks
    (taken), 8 x 32 x 5 = 1280 (the tiled kernel); 256 keys (taken) against 257
    (tiled); the row blocks whose staged V rows fit the CUs at once: E = 64 past
    192 keys 768 (taken) against 1024 (tiled; 192 keys: taken), E = 128 at 256 keys
    512 against 768, at 160 keys 768 against 1024; E = 32 1024 blocks of 256 keys
    (taken).  Checked on the first and last heads."""
    g = torch.Generator().manual_seed(sq + sk)
    q, k, v = (torch.randn(b, n, h, d, generator=g).bfloat16().to(cuda) for n in (sq, sk, sk))
    out = flash_attn_func(q, k, v, causal=True)
    for hh in (0, h - 1):
        sel = slice(hh, hh + 1)
        ref = attention(values(q[:, :, sel]), values(k[:, :, sel]), values(v[:, :, sel]), d ** -0.5, True)
        assert_close(out[:, :, sel], ref, torch.bfloat16, paged=False)
