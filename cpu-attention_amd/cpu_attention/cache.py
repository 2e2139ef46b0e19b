# Derived from ducviet00/cpu-attention (cpu_attention/cache.py), Apache License
# 2.0; modified for the MI355X build (see NOTICE at the repository root).  Kept
# from the original because the drop-in contract needs them: the function name
# and signature, the order of the argument checks, the exception types and the
# error messages.

"""``reshape_and_cache``: writing tokens into the paged KV cache.

The cache is in the original library's own layout -- per (block, head) a page of
``page_block_size`` tokens, K stored transposed inside the page -- so only this
library writes it: here, or through ``flash_attn_with_kvcache(k=..., v=...)``.
"""

import torch

from . import _kernel as K


def reshape_and_cache(key, value, k_cache, v_cache, slot_mapping) -> None:
    """Stores token ``i`` of ``key``/``value`` in cache slot ``slot_mapping[i]``.

    ``key`` and ``value`` are ``[num_tokens, nheads, headdim]`` with heads and head
    dims packed and any token stride (so the K and V slices of a fused projection
    are read in place); the caches are ``[num_blocks, nheads, page_block_size,
    headdim]``.  A slot ``s`` (int64) names block ``s // page_block_size``, position
    ``s % page_block_size``; a negative slot leaves its token out (padding), vLLM's
    convention.  The copy is queued on torch's current stream.
    """
    store = K.module().store
    if store(K.runtime(), key, value, k_cache, v_cache, slot_mapping) is None:
        key, value, slot_mapping = _check(key, value, k_cache, v_cache, slot_mapping)
        if store(K.runtime(), key, value, k_cache, v_cache, slot_mapping) is None:
            raise RuntimeError("cpu_attention: the kernel declined arguments that passed validation")


def _check(key, value, k_cache, v_cache, slots):
    """Called once the kernel module declined a store: raises the error that names
    the broken rule (the original library's checks in its order, then this
    build's device and alignment rules), or returns key, value and the slots in
    layouts the store kernel reads in place."""
    if key.dim() != 3 or value.shape != key.shape:
        raise ValueError("cpu_attention: key/value must both be [num_tokens, nheads, headdim]")
    if k_cache.dim() != 4 or v_cache.shape != k_cache.shape:
        raise ValueError("cpu_attention: k_cache/v_cache must be "
                         "[num_blocks, nheads, page_block_size, headdim] and match")
    if key.shape[1:] != (k_cache.shape[1], k_cache.shape[3]):
        raise ValueError("cpu_attention: key/value heads or head_dim do not match the cache")
    if not (k_cache.is_contiguous() and v_cache.is_contiguous()):
        raise ValueError("cpu_attention: the paged caches must be contiguous")
    if key.dtype not in K.DTYPES or not key.dtype == value.dtype == k_cache.dtype == v_cache.dtype:
        raise ValueError("cpu_attention: key/value and the caches must share a dtype (fp32 or bf16)")
    if key.shape[2] not in K.HEAD_DIMS or k_cache.shape[2] % 16:
        raise ValueError("cpu_attention: head_dim must be 32/64/128 and the page a multiple of 16")
    if slots.dtype != torch.int64 or slots.shape != (key.shape[0],):
        raise ValueError("cpu_attention: slot_mapping must be int64 [num_tokens]")
    capacity = k_cache.shape[0] * k_cache.shape[2]
    if key.shape[0] and int(slots.max()) >= capacity:
        raise ValueError("cpu_attention: slot_mapping points past the end of the cache")
    dev = k_cache.device
    if not (k_cache.is_cuda and v_cache.device == dev and key.device == dev and value.device == dev):
        raise ValueError("cpu_attention: the MI355X build takes tensors on one ROCm GPU")
    if not (K.aligned(k_cache) and K.aligned(v_cache)):
        raise ValueError("cpu_attention: the paged caches must start 16-byte aligned")
    plain = (torch.Tensor, torch.nn.Parameter)
    key, value, slots = (x if type(x) in plain else x.as_subclass(torch.Tensor) for x in (key, value, slots))
    # one shared layout with packed heads, then 16-byte alignment
    if key.stride(-1) != 1 or key.stride(-2) != key.shape[2] or value.stride() != key.stride():
        key, value = key.contiguous(), value.contiguous()
    step = key.stride(0) if key.shape[0] > 1 else 0
    if not (K.aligned(key, (step,)) and K.aligned(value, (step,))):
        key, value = (x.clone(memory_format=torch.contiguous_format) for x in (key, value))
    return key, value, slots.contiguous()
