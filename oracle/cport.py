"""ctypes access to ``libca_oracle.so``, the fp32 C port of the reference's CPU
algorithms (``ca_oracle.c``).

TEST INFRASTRUCTURE / CPU BASELINE (see oracle/__init__.py).  ``build()`` compiles it
with the Makefile beside this file.  Every function takes and returns numpy arrays
(bf16 as uint16 bit patterns).
"""

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB = os.path.join(HERE, "libca_oracle.so")
_LIB = []


def build():
    subprocess.run(["make", "-s", "-C", HERE], check=True)
    return LIB


def lib():
    if not _LIB:
        if not os.path.exists(LIB):
            build()
        h = ctypes.CDLL(LIB)
        vp, i64, i32, f32 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_float
        h.oracle_store.argtypes = [vp, vp, i64, vp, vp, vp, i64, i64, i64, i64, i64, i32]
        h.oracle_store.restype = None
        h.oracle_decode.argtypes = [i32, vp, i64, vp, vp, vp, vp, i64, i64, i64, i64, i64, f32, vp, i32]
        h.oracle_decode.restype = None
        h.oracle_flash.argtypes = [i32, vp, vp, vp, vp, i64, i64, i64, i64, i64, vp, vp, vp, f32, i32, i32]
        h.oracle_flash.restype = None
        h.oracle_max_threads.argtypes = []
        h.oracle_max_threads.restype = i32
        _LIB.append(h)
    return _LIB[0]


def _ptr(a):
    return a.ctypes.data_as(ctypes.c_void_p)


def max_threads():
    return lib().oracle_max_threads()


def store(kc, vc, key, value, slots, page, threads=0):
    """kc/vc uint32 word arrays [NB, H, P*W] (modified in place); key/value uint32
    [T, H, W] (contiguous); slots int64 [T]."""
    key = np.ascontiguousarray(key, np.uint32)
    value = np.ascontiguousarray(value, np.uint32)
    slots = np.ascontiguousarray(slots, np.int64)
    nb, heads, pw = kc.shape
    words = pw // page
    assert kc.flags.c_contiguous and vc.flags.c_contiguous
    lib().oracle_store(_ptr(key), _ptr(value), heads * words, _ptr(kc), _ptr(vc), _ptr(slots),
                       len(slots), heads, words, page, nb, threads)
    return kc, vc


def decode(q, kc, vc, lens, page_table, page, scale, bf16, threads=0):
    """q element array [N, H, E] (float32, or uint16 bf16 bits); caches as element
    arrays [NB, H, P, E] of the same kind.  Returns the output [N, H, E]."""
    q = np.ascontiguousarray(q)
    kc = np.ascontiguousarray(kc)
    vc = np.ascontiguousarray(vc)
    lens = np.ascontiguousarray(lens, np.int32)
    table = np.ascontiguousarray(page_table, np.int32)
    n, heads, hd = q.shape
    out = np.empty_like(q)
    lib().oracle_decode(1 if bf16 else 0, _ptr(q), heads * hd, _ptr(kc), _ptr(vc), _ptr(lens),
                        _ptr(table), table.shape[1], n, heads, hd, page, float(scale), _ptr(out),
                        threads)
    return out


def flash(q, k, v, scale, causal, bf16, threads=0):
    """q [B, L, H, E], k/v [B, S, H, E] element arrays (float32 or uint16 bf16
    bits, any strides numpy allows).  Returns the output [B, L, H, E]."""
    b, sq, heads, hd = q.shape
    assert hd % 16 == 0, "the C port tiles head_dim by 16"
    sk = k.shape[1]
    es = q.itemsize
    qs, ks, vs = ((ctypes.c_int64 * 3)(*[s // es for s in x.strides[:3]]) for x in (q, k, v))
    out = np.empty((b, sq, heads, hd), dtype=q.dtype)
    lib().oracle_flash(1 if bf16 else 0, _ptr(q), _ptr(k), _ptr(v), _ptr(out), b, sq, sk, heads, hd,
                       qs, ks, vs, float(scale), 1 if causal else 0, threads)
    return out
