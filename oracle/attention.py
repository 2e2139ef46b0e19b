"""Float64 eager attention and the tolerance gates.

TEST INFRASTRUCTURE (see oracle/__init__.py).  Restates ducviet00/cpu-attention
``tests/reference.py``: ``attention`` (:7-21) is matmul, additive bottom-right causal
mask, softmax, matmul in float64, with a row that sees no key equal to 0;
``check`` (:24-40) returns the reference's error measure and limit.  ``gate`` adds
the MI355X build's own gates (1e-5 relative for fp32, 2e-2 absolute for bf16).
"""

import numpy as np

FP32, BF16 = "fp32", "bf16"


def attention(q, k, v, scale, causal=False):
    """q [b, sq, h, d], k/v [b, sk, h, d] (MHA) -> float64 [b, sq, h, d].

    ``causal`` is bottom-right aligned: query i sees keys j <= i + sk - sq
    (reference.py:16-19); a row that sees no key is 0 (reference.py:20).
    """
    q, k, v = (np.asarray(x, np.float64).transpose(0, 2, 1, 3) for x in (q, k, v))  # [b, h, s, d]
    w = np.matmul(q, k.transpose(0, 1, 3, 2)) * float(scale)
    sq, sk = q.shape[2], k.shape[2]
    if causal:
        masked = np.arange(sk)[None, :] > np.arange(sq)[:, None] + sk - sq
        w = np.where(masked, -np.inf, w)
    m = w.max(axis=-1, keepdims=True, initial=-np.inf)  # no keys at all: an empty row
    empty = ~np.isfinite(m)
    e = np.exp(w - np.where(empty, 0.0, m))
    s = e.sum(axis=-1, keepdims=True)
    p = np.where(s > 0, e / np.where(s > 0, s, 1.0), 0.0)
    return np.ascontiguousarray(np.matmul(p, v).transpose(0, 2, 1, 3))


def check(got, ref, dtype, paged=False):
    """(max error, limit) of ``got`` against the float64 ``ref`` (reference.py:24-40).

    flash fp32 2e-4, flash bf16 3e-2, paged fp32 1e-6; paged bf16 is 1e-3 beyond
    the unavoidable rounding of the exact result to bf16.
    """
    from .bf16 import round_float

    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    err = np.abs(got - ref)
    if dtype == FP32:
        return float(err.max(initial=0.0)), (1e-6 if paged else 2e-4)
    if not paged:
        return float(err.max(initial=0.0)), 3e-2
    rounding = np.abs(ref - round_float(ref.astype(np.float32)).astype(np.float64))
    return float((err - rounding).max(initial=0.0)), 1e-3


def gate(got, ref, dtype):
    """The MI355X build's gate: fp32 max|got-ref| <= 1e-5 * max(1, max|ref|);
    bf16 max|got-ref| <= 2e-2.  Returns (error, limit)."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    err = float(np.abs(got - ref).max(initial=0.0))
    if dtype == FP32:
        return err, 1e-5 * max(1.0, float(np.abs(ref).max(initial=0.0)))
    return err, 2e-2
