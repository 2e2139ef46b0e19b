"""Pins for the CPU oracle (CPU only).

The reference ships no golden vectors for this path (its tests compare against a
float64 eager oracle computed at test time, tests/reference.py), so each oracle
function is pinned here against something other than itself:

* ``attention``: torch's float64 scaled_dot_product_attention (an independent
  library routine, with an explicit bottom-right mask), plus closed forms a
  dropped term, a wrong sign or a transposed operand would break (one key ->
  that key's value; q = 0 -> mean of V; a dominant logit -> its value; zero
  rows; key-permutation invariance);
* ``check`` / ``gate``: known answers at and just past each limit;
* ``bf16``: torch's ``.bfloat16()`` on ties, NaN, inf, subnormals and randoms;
* ``layout``: the reference's element-level statement of the layout
  (paged_attn.mojo:76-82, :111-113; a different formula from the oracle's word
  indexing) on a hand-sized example, the reference's 16x16 word-transpose block
  store (:117-130) as a second implementation, store/gather round trips, and the
  reference test's "reshape_and_cache writes what the append writes"
  (tests/test_kvcache.py:143-161);
* ``cport``: byte equality with ``layout.store`` and the gates against the
  float64 oracle, including the inputs of the reference's native Mojo test
  (its LCG, cpu_attention/_mojo/tests/test_attention.mojo:15-21).
"""

import numpy as np
import pytest
import torch

from oracle import bf16, cport, layout
from oracle.attention import BF16, FP32, attention, check, gate


def _sdpa(q, k, v, scale, causal):
    """torch float64 SDPA with the bottom-right mask as an explicit boolean mask."""
    qt, kt, vt = (torch.from_numpy(np.asarray(x, np.float64)).transpose(1, 2) for x in (q, k, v))
    sq, sk = qt.shape[2], kt.shape[2]
    mask = None
    if causal:
        mask = torch.arange(sk)[None, :] <= torch.arange(sq)[:, None] + sk - sq
    out = torch.nn.functional.scaled_dot_product_attention(qt, kt, vt, attn_mask=mask, scale=scale)
    out = torch.nan_to_num(out, 0.0)  # rows with no visible key
    if causal:
        empty = ~mask.any(-1)
        out[:, :, empty] = 0.0
    return out.transpose(1, 2).numpy()


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("sq,sk", [(1, 1), (7, 7), (5, 13), (13, 5), (1, 40), (33, 33)])
def test_attention_matches_torch_sdpa(sq, sk, causal):
    rng = np.random.default_rng(sq * 100 + sk)
    b, h, d = 2, 3, 16
    q, k, v = (rng.standard_normal((b, n, h, d)) for n in (sq, sk, sk))
    got = attention(q, k, v, 0.3, causal)
    np.testing.assert_allclose(got, _sdpa(q, k, v, 0.3, causal), rtol=1e-12, atol=1e-12)


def test_attention_closed_forms():
    rng = np.random.default_rng(0)
    k, v = rng.standard_normal((1, 9, 2, 8)), rng.standard_normal((1, 9, 2, 8))
    # one key: the output is that key's value, whatever q and the scale are
    q = rng.standard_normal((1, 4, 2, 8))
    np.testing.assert_allclose(attention(q, k[:, :1], v[:, :1], 0.7), np.broadcast_to(v[:, :1], q.shape))
    # q = 0: uniform weights, the output is the mean of V
    np.testing.assert_allclose(attention(np.zeros((1, 3, 2, 8)), k, v, 1.0),
                               np.broadcast_to(v.mean(1, keepdims=True), (1, 3, 2, 8)), atol=1e-14)
    # a dominant logit selects its key's value (q parallel to key 5, huge scale)
    qd = np.repeat(k[:, 5:6], 1, axis=1)
    out = attention(qd, k, v, 1e3)
    np.testing.assert_allclose(out[0, 0], v[0, 5], atol=1e-9)
    # causal with sq > sk: the first sq - sk rows see nothing and are exactly 0
    out = attention(rng.standard_normal((1, 6, 2, 8)), k[:, :2], v[:, :2], 0.5, causal=True)
    assert np.all(out[:, :4] == 0) and np.all(out[:, 4:] != 0)
    # bottom-right: the last row sees every key, so it equals the non-causal row
    q6 = rng.standard_normal((1, 6, 2, 8))
    np.testing.assert_allclose(attention(q6, k, v, 0.5, True)[:, -1], attention(q6, k, v, 0.5)[:, -1])
    # row 0 of an sq = sk causal call sees only key 0
    np.testing.assert_allclose(attention(q6, k[:, :6], v[:, :6], 0.5, True)[:, 0], v[:, 0])
    # no keys at all (a zero-length cache): the row is 0
    assert np.all(attention(q, k[:, :0], v[:, :0], 0.5) == 0)
    # non-causal attention ignores the order of the keys
    perm = rng.permutation(9)
    np.testing.assert_allclose(attention(q, k, v, 0.4), attention(q, k[:, perm], v[:, perm], 0.4),
                               atol=1e-13)


def test_check_limits():
    ref = np.array([0.5, -1.25, 3.0])
    assert check(ref + 1e-6, ref, FP32, paged=True) == pytest.approx((1e-6, 1e-6))
    err, tol = check(ref + 2e-6, ref, FP32, paged=True)
    assert err > tol
    assert check(ref + 1e-4, ref, FP32)[1] == 2e-4
    assert check(ref + 1e-2, ref, BF16)[1] == 3e-2
    # paged bf16 measures the error beyond rounding the exact result to bf16:
    # the rounded result itself scores 0.
    exact = np.array([0.1, 0.2, 1 / 3, -2.7182818])
    rounded = bf16.round_float(exact.astype(np.float32)).astype(np.float64)
    err, tol = check(rounded, exact, BF16, paged=True)
    assert err <= 1e-12 and tol == 1e-3
    err, _ = check(rounded + 2e-3, exact, BF16, paged=True)
    assert err > 1e-3
    # the MI355X gates
    assert gate(ref + 2.9e-5, ref, FP32)[0] <= gate(ref + 2.9e-5, ref, FP32)[1]  # 1e-5 * 3
    err, tol = gate(ref + 3.1e-5, ref, FP32)
    assert err > tol
    assert gate(ref + 1e-2, ref, BF16) == pytest.approx((1e-2, 2e-2))


def test_bf16_matches_torch():
    rng = np.random.default_rng(1)
    x = np.concatenate([
        rng.standard_normal(4096).astype(np.float32) * 10,
        np.array([0.0, -0.0, 1.0, 1.00390625, 1.005859375, 1.0078125, 3.0e38, -3.0e38,
                  1e-40, -1e-40, np.inf, -np.inf], np.float32),
        # exact ties between two bf16 values: round to the even one
        (np.arange(1, 200, dtype=np.uint32) << 16 | 0x8000).view(np.float32),
    ])
    want = torch.from_numpy(x).bfloat16().view(torch.int16).numpy().view(np.uint16)
    np.testing.assert_array_equal(bf16.from_float(x), want)
    np.testing.assert_array_equal(bf16.to_float(want), torch.from_numpy(want.view(np.int16)).view(
        torch.bfloat16).float().numpy())
    assert np.isnan(bf16.to_float(bf16.from_float(np.array([np.nan], np.float32))))[0]


def _element_cache(kc_words, dtype):
    return layout.elements_of(kc_words, dtype)


@pytest.mark.parametrize("dtype", [FP32, BF16])
def test_layout_element_statement(dtype):
    """The reference states the layout per element (paged_attn.mojo:76-82, 90-94,
    111-113); the oracle indexes 32-bit words.  One token, values = dim index + 1."""
    nb, heads, page, hd = 3, 2, 16, 32
    words = layout.words_per_token(hd, dtype)
    kc = np.zeros((nb, heads, page * words), np.uint32)
    vc = np.zeros_like(kc)
    vals = np.arange(1, hd + 1, dtype=np.float32)
    bits = bf16.from_float(vals) if dtype == BF16 else vals
    key = np.zeros((1, heads, hd), bits.dtype)
    key[0, 1] = bits  # head 1 only
    slot = 1 * page + 5  # block 1, position 5
    layout.store(kc, vc, layout.words_of(key, dtype), layout.words_of(key, dtype),
                 np.array([slot]), page)
    kel = _element_cache(kc, dtype).reshape(-1)
    vel = _element_cache(vc, dtype).reshape(-1)
    block = (1 * heads + 1) * page * hd  # element where block (1, head 1) starts
    for d in range(hd):
        if dtype == BF16:
            kpos = block + ((d // 2) * page + 5) * 2 + (d & 1)  # :76-82
        else:
            kpos = block + d * page + 5  # :90-94
        assert kel[kpos] == bits[d]
        assert vel[block + 5 * hd + d] == bits[d]  # :111-113
    # nothing else was written
    assert np.count_nonzero(kel) == hd and np.count_nonzero(vel) == hd


def _store_k_block(kc, key_words, slot0, page):
    """The reference's consecutive-slot path: 16 tokens in consecutive slots of one
    page, K written through a 16x16 transpose of 32-bit words (store_k_block,
    paged_attn.mojo:117-130), independent of ``layout.store``'s indexing."""
    nb, heads, pw = kc.shape
    words = pw // page
    blk, t0 = slot0 // page, slot0 % page
    flat = kc.reshape(-1)
    for h in range(heads):
        base = (blk * heads + h) * page * words
        for w0 in range(0, words, 16):
            tile = key_words[:16, h, w0:w0 + 16]  # rows = tokens, cols = words
            tr = tile.T  # rows = words
            for j in range(16):
                flat[base + (w0 + j) * page + t0: base + (w0 + j) * page + t0 + 16] = tr[j]


@pytest.mark.parametrize("dtype,hd,page", [(FP32, 32, 16), (BF16, 64, 32), (BF16, 128, 48)])
def test_layout_block_transpose_path(dtype, hd, page):
    rng = np.random.default_rng(hd + page)
    nb, heads = 4, 3
    words = layout.words_per_token(hd, dtype)
    key = rng.integers(0, 2**32, size=(16, heads, words), dtype=np.uint32)
    slot0 = 2 * page + 16  # consecutive slots, one page
    a = np.zeros((nb, heads, page * words), np.uint32)
    layout.store(a, np.zeros_like(a), key, key, np.arange(slot0, slot0 + 16), page)
    b = np.zeros_like(a)
    _store_k_block(b, key, slot0, page)
    np.testing.assert_array_equal(a, b)


@pytest.mark.parametrize("dtype", [FP32, BF16])
def test_layout_round_trip_and_append_equivalence(dtype):
    rng = np.random.default_rng(5)
    page, heads, hd = 16, 2, 64
    words = layout.words_per_token(hd, dtype)
    lens = [70, 5, 33]
    npages = [-(-n // page) for n in lens]
    nb = sum(npages) + 2
    order = rng.permutation(nb)
    table = np.full((len(lens), max(npages) + 1), order[-1], np.int64)
    start = 0
    for i, n in enumerate(npages):
        table[i, :n] = order[start:start + n]
        start += n
    toks = [rng.integers(0, 2**32, size=(n, heads, words), dtype=np.uint32) for n in lens]
    # path 1: one reshape_and_cache over all tokens, with padding slots (-1)
    slots = np.concatenate([layout.prompt_slots(0, n, table[i], page) for i, n in enumerate(lens)]
                           + [np.full(3, -1)])
    allk = np.concatenate(toks + [rng.integers(0, 2**32, size=(3, heads, words), dtype=np.uint32)])
    k1 = np.zeros((nb, heads, page * words), np.uint32)
    v1 = np.zeros_like(k1)
    layout.store(k1, v1, allk, allk[::-1].copy(), slots, page)
    # path 2: token by token through the append (position = current length)
    k2, v2 = np.zeros_like(k1), np.zeros_like(k1)
    vals = allk[::-1]
    flat_v = {}
    i0 = 0
    for i, n in enumerate(lens):
        for t in range(n):
            s = layout.append_slots([t], table[i:i + 1], page)
            layout.store(k2, v2, toks[i][t:t + 1], vals[i0 + t:i0 + t + 1], s, page)
        flat_v[i] = vals[i0:i0 + n]
        i0 += n
    np.testing.assert_array_equal(k1, k2)
    np.testing.assert_array_equal(v1, v2)
    # round trip: gather returns exactly what was stored
    for i, n in enumerate(lens):
        kg, vg = layout.gather(k1, v1, table[i], n, page)
        np.testing.assert_array_equal(kg, toks[i])
        np.testing.assert_array_equal(vg, flat_v[i])
    # negative lengths and positions past the table store nothing
    assert list(layout.append_slots([-1, 10**6], table[:2], page)) == [-1, -1]


def _lcg(n, seed):
    """The reference's native-test inputs (test_attention.mojo:15-21)."""
    out = np.empty(n, np.float32)
    s = seed
    for i in range(n):
        s = (s * 1103515245 + 12345) % 2147483648
        out[i] = np.float32((s % 2001 - 1000) / 1000.0)
    return out, s


@pytest.mark.parametrize("dtype", [FP32, BF16])
@pytest.mark.parametrize("page", [16, 32, 48, 64])
def test_cport_decode_against_float64(dtype, page):
    """The C port on the reference native test's case shape: 2 sequences, 4 heads,
    hd 64, lengths ending mid-tile, LCG inputs, scale 0.125, reversed page order."""
    heads, hd = 4, 64
    lens = [page * 3 + 5, 2 * page - 1]
    tokens = sum(lens)
    kn, s = _lcg(tokens * heads * hd, 7)
    vn, s = _lcg(tokens * heads * hd, s)
    q, s = _lcg(2 * heads * hd, s)
    pages_per = -(-max(lens) // page)
    table = np.array([[si * pages_per + (pages_per - 1 - p) for p in range(pages_per)] for si in range(2)])
    slots = np.concatenate([table[si][np.arange(n) // page] * page + np.arange(n) % page
                            for si, n in enumerate(lens)])
    words = layout.words_per_token(hd, dtype)
    to_bits = (lambda x: bf16.from_float(x)) if dtype == BF16 else (lambda x: x)
    kw = layout.words_of(to_bits(kn).reshape(tokens, heads, hd), dtype)
    vw = layout.words_of(to_bits(vn).reshape(tokens, heads, hd), dtype)
    kc = np.zeros((2 * pages_per, heads, page * words), np.uint32)
    vc = np.zeros_like(kc)
    kc2, vc2 = kc.copy(), vc.copy()
    layout.store(kc, vc, kw, vw, slots, page)
    cport.store(kc2, vc2, kw, vw, slots, page)
    np.testing.assert_array_equal(kc, kc2)
    np.testing.assert_array_equal(vc, vc2)
    qb = to_bits(q).reshape(2, heads, hd)
    qv = bf16.to_float(qb) if dtype == BF16 else qb
    ref = layout.decode(qv, kc, vc, table, lens, 0.125, page, dtype)
    shape = (kc.shape[0], heads, page, hd)
    got = cport.decode(qb, layout.elements_of(kc, dtype).reshape(shape),
                       layout.elements_of(vc, dtype).reshape(shape), lens, table, page, 0.125,
                       dtype == BF16, threads=2)
    got = bf16.to_float(got) if dtype == BF16 else got
    # the native test's gates (test_attention.mojo:93) and the reference pytest gates
    assert np.abs(got - ref).max() <= (1e-5 if dtype == FP32 else 2e-2)
    err, tol = check(got, ref, dtype, paged=True)
    assert err <= tol


@pytest.mark.parametrize("dtype", [FP32, BF16])
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("sq,sk", [(1, 1), (37, 100), (100, 37), (129, 129)])
@pytest.mark.parametrize("tiles", ["host", "avx2"])
def test_cport_flash_against_float64(dtype, causal, sq, sk, tiles, monkeypatch):
    if tiles == "avx2":  # the AVX2 tiles, whatever the host has
        monkeypatch.setenv("CA_ORACLE_AVX2", "1")
    rng = np.random.default_rng(sq * 7 + sk)
    b, h, hd = 2, 3, 64
    q, k, v = (rng.standard_normal((b, n, h, hd)).astype(np.float32) for n in (sq, sk, sk))
    if dtype == BF16:
        q, k, v = (bf16.from_float(x) for x in (q, k, v))
        vals = [bf16.to_float(x) for x in (q, k, v)]
    else:
        vals = [q, k, v]
    ref = attention(*vals, hd ** -0.5, causal)
    got = cport.flash(q, k, v, hd ** -0.5, causal, dtype == BF16, threads=2)
    got = bf16.to_float(got) if dtype == BF16 else got
    err, tol = check(got, ref, dtype)
    assert err <= tol
    # the plausible-mistake check: a top-left causal mask would fail this case
    if causal and sq != sk:
        wrong = attention(*vals, hd ** -0.5, False)
        assert np.abs(wrong - ref).max() > tol
