"""The paged KV-cache layout, its writers and paged decode, in numpy.

TEST INFRASTRUCTURE (see oracle/__init__.py).  Restates ducviet00/cpu-attention
``cpu_attention/_mojo/src/paged_attn.mojo`` (x86 mapping, ``V_PAIRS_ARM = False``):

* ``PageLayout`` (:58-130): caches are ``[num_blocks, heads, page, head_dim]``
  elements; block (b, h) starts at element (b*H + h)*P*E.  Working in 32-bit
  words (fp32: one element; bf16: the pair of dims (2*d2, 2*d2+1), low half first),
  a head's K row is W words and sits *transposed* in the block: word (w, t) at
  w*P + t (store_token :72-95, store_k_block :117-130); V rows are not
  transposed: word (t, w) at t*W + w (store_v :99-113).
* the store (:151-204, :822-851): token i goes to slot s = slots[i], block s // P,
  position s % P; s < 0 skips the token.  The append (:165-170) stores at position
  lens[s] through the block table; lens < 0 skips.
* decode (:714-782): the row attends its first ``len`` cached keys; zero keys
  give 0 (:307-310).

All caches here are numpy uint32 *word* arrays of shape [NB, H, P*W]; use
``words_of`` / ``elements_of`` to move between element tensors and words.
"""

import numpy as np

from .attention import attention


def words_per_token(head_dim, dtype):
    return head_dim // 2 if dtype == "bf16" else head_dim


def words_of(bits, dtype):
    """Element bit patterns (uint16 for bf16, float32/uint32 for fp32) whose last
    axis is head_dim -> uint32 words, last axis W."""
    a = np.ascontiguousarray(bits)
    if dtype == "bf16":
        return a.astype(np.uint16).view(np.uint32)
    return a.view(np.uint32) if a.dtype != np.uint32 else a


def elements_of(words, dtype):
    """Inverse of ``words_of``: uint16 bit patterns (bf16) or float32 (fp32)."""
    w = np.ascontiguousarray(words, np.uint32)
    return w.view(np.uint16) if dtype == "bf16" else w.view(np.float32)


def k_index(blk, h, t, w, heads, page, words):
    """Flat word index of K word w of the token at position t of block blk, head h."""
    return ((blk * heads + h) * words + w) * page + t


def v_index(blk, h, t, w, heads, page, words):
    """Flat word index of V word w of the token at position t of block blk, head h."""
    return ((blk * heads + h) * page + t) * words + w


def store(kc, vc, key, value, slots, page):
    """reshape_and_cache on word arrays: kc/vc [NB, H, P*W], key/value [T, H, W],
    slots int64 [T].  Negative slots (and, as a guard, slots past the cache) are
    skipped.  Modifies kc/vc in place and returns them."""
    nb, heads, pw = kc.shape
    words = pw // page
    slots = np.asarray(slots, np.int64)
    ok = (slots >= 0) & (slots < nb * page)
    blk, off = slots[ok] // page, slots[ok] % page
    k4 = kc.reshape(nb, heads, words, page)
    v4 = vc.reshape(nb, heads, page, words)
    k4[blk, :, :, off] = np.asarray(key)[ok]
    v4[blk, :, off, :] = np.asarray(value)[ok]
    return kc, vc


def append_slots(lens, page_table, page):
    """The slots the decode-time append writes (paged_attn.mojo:165-170): position
    lens[s] of sequence s through its page-table row; -1 where lens < 0 or the
    position is beyond the table."""
    lens = np.asarray(lens, np.int64)
    table = np.asarray(page_table, np.int64)
    cap = table.shape[1] * page
    ok = (lens >= 0) & (lens < cap)
    col = np.where(ok, lens // page, 0)
    slots = table[np.arange(len(lens)), col] * page + lens % page
    return np.where(ok, slots, -1)


def prompt_slots(start, n, page_table_row, page):
    """Slots of positions start .. start+n-1 of one sequence (the multi-token
    append, flash_attn_interface.py:109-117)."""
    pos = np.arange(start, start + n, dtype=np.int64)
    return np.asarray(page_table_row, np.int64)[pos // page] * page + pos % page


def gather(kc, vc, page_table_row, length, page):
    """Dense K/V words [length, H, W] of one sequence, read back through its page
    table (the inverse of ``store``)."""
    nb, heads, pw = kc.shape
    words = pw // page
    t = np.arange(length, dtype=np.int64)
    blk = np.asarray(page_table_row, np.int64)[t // page]
    off = t % page
    k4 = kc.reshape(nb, heads, words, page)
    v4 = vc.reshape(nb, heads, page, words)
    return k4[blk, :, :, off], v4[blk, :, off, :]


def to_values(words, dtype):
    """uint32 words [..., W] -> float64 element values [..., E]."""
    from .bf16 import to_float

    e = elements_of(words, dtype)
    return (to_float(e) if dtype == "bf16" else e).astype(np.float64)


def decode(q, kc, vc, page_table, lens, scale, page, dtype):
    """Paged decode oracle: q values [N, H, E] -> float64 [N, H, E].  Each row
    attends the first lens[s] keys of its sequence; lens <= 0 gives 0."""
    q = np.asarray(q, np.float64)
    n, heads, e = q.shape
    out = np.zeros((n, heads, e))
    for s in range(n):
        ln = int(lens[s])
        if ln <= 0:
            continue
        kw, vw = gather(kc, vc, page_table[s], ln, page)
        k, v = to_values(kw, dtype), to_values(vw, dtype)  # [len, H, E]
        out[s] = attention(q[s][None, None], k[None], v[None], scale)[0, 0]
    return out
