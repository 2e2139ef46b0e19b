"""Writing the paged KV cache.

The cache layout is the reference's own (head-major, K transposed inside the page;
cpu_attention/_mojo/src/paged_attn.mojo:58-130 of ducviet00/cpu-attention), so only
this library writes it: ``reshape_and_cache`` (vLLM's signature), or
``flash_attn_with_kvcache(k=..., v=...)``.
"""

import torch

from . import _kernel as K


def reshape_and_cache(key, value, k_cache, v_cache, slot_mapping) -> None:
    """Scatter K/V of ``num_tokens`` tokens into the paged cache.

    ``key``/``value`` are ``[num_tokens, nheads, headdim]`` (any token stride;
    heads and dims contiguous, so chunks of a fused projection work as is), the
    caches ``[num_blocks, nheads, page_block_size, headdim]``. Token ``i`` goes to
    slot ``slot_mapping[i]`` (int64): page ``slot // page_block_size``, position
    ``slot % page_block_size``; a negative slot skips the token (padding).
    The copy is enqueued on torch's current stream.
    """
    if K.module().store(K.runtime(), key, value, k_cache, v_cache, slot_mapping) is None:
        key, value, slot_mapping = _check(key, value, k_cache, v_cache, slot_mapping)
        if K.module().store(K.runtime(), key, value, k_cache, v_cache, slot_mapping) is None:
            raise RuntimeError("cpu_attention: the kernel declined arguments that passed validation")


def _check(key, value, k_cache, v_cache, slots):
    """Raise the precise error for a call the kernels declined, or return key/value
    and the slots in layouts they read in place (the reference's checks, cache.py:28-52,
    then the GPU build's: one device, 16-byte alignment)."""
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
    if key.shape[0] and int(slots.max()) >= k_cache.shape[0] * k_cache.shape[2]:
        raise ValueError("cpu_attention: slot_mapping points past the end of the cache")
    dev = k_cache.device
    if not (k_cache.is_cuda and v_cache.device == dev and key.device == dev and value.device == dev):
        raise ValueError("cpu_attention: the MI355X build takes tensors on one ROCm GPU")
    if not (K.aligned(k_cache) and K.aligned(v_cache)):
        raise ValueError("cpu_attention: the paged caches must start 16-byte aligned")
    key, value, slots = (x.as_subclass(torch.Tensor) if type(x) not in (torch.Tensor, torch.nn.Parameter)
                         else x for x in (key, value, slots))
    if not (key.stride(-1) == 1 and key.stride(-2) == key.shape[2] and value.stride() == key.stride()):
        key, value = key.contiguous(), value.contiguous()
    tstride = key.stride(0) if key.shape[0] > 1 else 0
    if not (K.aligned(key, (tstride,)) and K.aligned(value, (tstride,))):
        key, value = (x.clone(memory_format=torch.contiguous_format) for x in (key, value))
    return key, value, slots.contiguous()
