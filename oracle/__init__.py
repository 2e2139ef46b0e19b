"""CPU oracle for cpu-attention's three ops -- TEST INFRASTRUCTURE, NOT PRODUCT CODE.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline``
leg may import or run anything in this package, and only as the checker (or, for
the C port, as the timed CPU baseline); the GPU path never routes through it.

Contents (each function cites the reference file:line it restates):

* ``attention`` -- float64 eager attention with bottom-right causal masking and
  zero rows, and the tolerance gates (``check``, ``gate``): a restatement of
  ducviet00/cpu-attention ``tests/reference.py:7-40``.
* ``layout`` -- the paged-cache byte layout as an index permutation, the
  slot-mapped scatter (``reshape_and_cache``), the decode-time append, the
  gather back to dense K/V, and paged decode on top of ``attention``:
  ``cpu_attention/_mojo/src/paged_attn.mojo:58-204, 714-782``.
* ``bf16`` -- fp32 <-> bf16 bit conversions (round to nearest even).
* ``cport`` -- ctypes access to ``ca_oracle.c``: an fp32 C port of the
  reference's CPU algorithms (paged decode with base-2 online softmax over
  key steps, blocked prefill, the store), parallelised with OpenMP; used as the
  CPU baseline and cross-checked against the float64 oracle.

How each part is pinned (checked against something other than itself) is listed
in ``tests/test_oracle.py``; nothing here is "parity unpinned".
"""
