# Derived from ducviet00/cpu-attention (cpu_attention/flash_attn_interface.py),
# Apache License 2.0; modified for the MI355X build (see NOTICE at the repository
# root).  Kept from the original because the drop-in contract needs them: the
# function names and signatures, which options are refused, the order of the
# argument checks, the exception types and the error messages.

"""The flash-attn entry points, computed on an MI355X.

``flash_attn_func`` (dense prefill) and ``flash_attn_with_kvcache`` (paged decode)
take flash-attn's arguments.  An option this build does not implement is refused
with ``NotImplementedError`` rather than ignored.  The fast path hands the
tensors straight to the kernel module, which checks them itself and returns
``None`` for anything its kernels cannot read; only then does this module
examine the arguments, to name what is wrong or to copy a tensor into a layout
the kernels can read.

Running on a GPU adds three rules: the tensors live on one ROCm GPU (index
tensors -- ``cache_seqlens``, ``page_table``, ``cache_batch_idx`` -- may also be
CPU tensors, and are copied over); a call returns once its kernels are queued on
torch's current stream; and an integer ``cache_seqlens`` or the positions of a
multi-token append are made on the GPU.
"""

import torch

from . import _kernel as K
from .cache import reshape_and_cache

_MHA_ONLY = "cpu_attention supports MHA only (nheads == nheads_k); GQA/MQA are not supported yet"
_DEVICE = "cpu_attention: the MI355X build takes tensors on one ROCm GPU"
_REFUSED = ("cpu_attention: qv, rotary, cache_leftpad, varlen, descale, sliding "
            "windows, softcap, attention_chunk, alibi and return_softmax_lse are not supported")
_ENTRIES = []  # [runtime handle, module decode, module flash] once the library is loaded


def _entries():
    if not _ENTRIES:
        mod = K.module()
        _ENTRIES.extend((K.runtime(), mod.decode, mod.flash))
    return _ENTRIES


def _as_plain(x):
    """Tensor subclasses become plain tensors (the kernel module reads plain
    tensors only); anything else passes through."""
    if isinstance(x, torch.Tensor) and type(x) not in (torch.Tensor, torch.nn.Parameter):
        return x.as_subclass(torch.Tensor)
    return x


def _in_place_or_copy(x, strides):
    """``x`` when its pointer and the given element strides keep the 16-byte
    alignment the kernels' vector loads need, else a contiguous copy."""
    return x if K.aligned(x, strides) else x.clone(memory_format=torch.contiguous_format)


def _heads_contiguous(x):
    """``x`` with its last two dims packed (heads x head_dim), copied if they are
    not; any leading stride is kept."""
    if x.stride(-1) != 1 or x.stride(-2) != x.shape[-1]:
        return x.contiguous()
    return _in_place_or_copy(x, (x.stride(0) if x.shape[0] > 1 else 0,))


def flash_attn_with_kvcache(
    q,
    k_cache,
    v_cache,
    k=None,
    v=None,
    qv=None,
    rotary_cos=None,
    rotary_sin=None,
    cache_seqlens=None,
    cache_batch_idx=None,
    cache_leftpad=None,
    page_table=None,
    cu_seqlens_q=None,
    cu_seqlens_k_new=None,
    max_seqlen_q=None,
    rotary_seqlens=None,
    q_descale=None,
    k_descale=None,
    v_descale=None,
    softmax_scale=None,
    causal=False,
    window_size=(-1, -1),
    attention_chunk=0,
    softcap=0.0,
    rotary_interleaved=True,
    scheduler_metadata=None,
    num_splits=0,
    pack_gqa=None,
    sm_margin=0,
    return_softmax_lse=False,
    block_table=None,
    alibi_slopes=None,
):
    """Attention of one new query token per sequence over that sequence's paged
    K/V cache.

    Shapes: ``q`` ``[batch, 1, nheads, headdim]`` with ``nheads_k == nheads``
    (grouped or multi-query heads are refused); the caches
    ``[num_blocks, nheads, page_block_size, headdim]`` in this library's layout
    (head-major blocks, K transposed inside a block), contiguous, written only by
    ``reshape_and_cache`` or by ``k``/``v`` here.  ``cache_seqlens`` holds each
    sequence's cached length (an int means the same for all); ``page_table``
    maps each sequence's logical pages to cache blocks (``block_table`` is
    accepted as its flash-attn 2 name, not both).

    ``k``/``v`` of ``n`` new tokens per sequence are written at positions
    ``cache_seqlens .. cache_seqlens + n - 1`` before the query attends, so the
    query then sees ``cache_seqlens + n`` keys.  ``causal`` changes nothing: the
    query is the newest position anyway.  ``softmax_scale`` defaults to
    ``headdim ** -0.5``.  ``num_splits``, ``pack_gqa``, ``scheduler_metadata``,
    ``sm_margin`` and ``rotary_interleaved`` are scheduling hints with no effect;
    rotary embedding, ``qv``, ``cache_leftpad``, the varlen arguments, descaling,
    sliding windows, softcap, ``attention_chunk``, ``alibi_slopes`` and
    ``return_softmax_lse`` raise ``NotImplementedError``.
    """
    refused = (qv, rotary_cos, rotary_sin, cache_leftpad, cu_seqlens_q, cu_seqlens_k_new, max_seqlen_q,
               rotary_seqlens, q_descale, k_descale, v_descale, alibi_slopes)
    if any(x is not None for x in refused) or window_size != (-1, -1) or softcap or attention_chunk \
            or return_softmax_lse:
        raise NotImplementedError(_REFUSED)
    if block_table is not None:
        if page_table is not None:
            raise ValueError("cpu_attention: pass `page_table` or `block_table`, not both")
        page_table = block_table
    if page_table is None:
        raise ValueError("cpu_attention: pass `page_table`")
    if cache_batch_idx is not None:
        # query s reads the cache rows of sequence cache_batch_idx[s]
        page_table = page_table.index_select(0, cache_batch_idx.to(page_table.device).long())
    if not isinstance(cache_seqlens, torch.Tensor):
        if cache_seqlens is None:
            raise ValueError("cpu_attention: `cache_seqlens` is required")
        where = q.device if isinstance(q, torch.Tensor) else "cpu"
        cache_seqlens = torch.full((q.shape[0],), cache_seqlens, dtype=torch.int32, device=where)
    if k is not None and k.shape[1] != 1:
        out = _append_prompt(q, k_cache, v_cache, k, v, cache_seqlens, page_table, softmax_scale)
        if out is not None:
            return out
        cache_seqlens, k, v = cache_seqlens + k.shape[1], None, None
    rt, decode, _ = _ENTRIES or _entries()
    out = decode(rt, q, k_cache, v_cache, k, v, None, cache_seqlens, page_table, softmax_scale, None)
    if out is None:
        q, k_cache, v_cache, k, v, page_table, cache_seqlens = _check_kvcache(
            q, k_cache, v_cache, k, v, page_table, cache_seqlens)
        out = decode(rt, q, k_cache, v_cache, k, v, None, cache_seqlens, page_table,
                     softmax_scale, None)
        if out is None:
            raise RuntimeError("cpu_attention: the kernel declined arguments that passed validation")
    return out


def _append_prompt(q, k_cache, v_cache, k, v, lens, page_table, scale):
    """Writes ``n = k.shape[1]`` new tokens per sequence at ``lens .. lens + n - 1``.

    The native path does the write and the decode in one call (the store kernel
    computes the slots from the page table) and returns the decode's output.
    Whatever it declines is written here through ``reshape_and_cache`` instead,
    and ``None`` is returned: the caller then decodes over ``lens + n`` keys, and
    its checks raise the precise error for a bad call.  Positions past the page
    table get slot -1 (nothing written) rather than an out-of-range gather; with
    host checks on, a prompt that does not fit is refused before any of it is
    written."""
    if isinstance(q, torch.Tensor) and isinstance(k, torch.Tensor):
        out = K.module().append_decode(K.runtime(), q, k_cache, v_cache, k, v, lens, page_table, scale)
        if out is not None:
            return out
    n, page = k.shape[1], k_cache.shape[2]
    if K.host_checks() and isinstance(lens, torch.Tensor) and lens.numel() \
            and isinstance(page_table, torch.Tensor) and page_table.dim() == 2 \
            and int(lens.max()) + n > page_table.shape[1] * page:
        raise ValueError("cpu_attention: cache_seqlens exceed the page table's capacity")
    dev = k.device
    table = page_table.to(dev).long()
    pos = lens.to(dev).long()[:, None] + torch.arange(n, device=dev)[None]
    fits = (pos >= 0) & (pos < table.shape[1] * page)
    blocks = table.gather(1, torch.where(fits, pos // page, torch.zeros_like(pos)))
    slots = torch.where(fits, blocks * page + pos % page, torch.full_like(pos, -1))
    reshape_and_cache(k.reshape(-1, *k.shape[2:]), v.reshape(-1, *v.shape[2:]), k_cache, v_cache,
                      slots.flatten())
    return None


def _check_kvcache(q, k_cache, v_cache, k, v, page_table, lens):
    """Called once the kernel module declined a decode: raises the error that
    names the broken rule (the original library's checks, in its order, then this
    build's device and alignment rules), or returns the arguments in layouts the
    kernels read in place."""
    q, k_cache, v_cache, k, v, page_table, lens = map(_as_plain, (q, k_cache, v_cache, k, v, page_table, lens))
    if q.dim() != 4:
        raise ValueError("cpu_attention: q must be [batch, 1, nheads, headdim]")
    if q.shape[1] != 1:
        raise NotImplementedError("cpu_attention decodes one query token per sequence")
    batch, _, heads, hd = q.shape
    if k_cache.dim() != 4 or v_cache.shape != k_cache.shape:
        raise ValueError("cpu_attention: k_cache/v_cache must be "
                         "[num_blocks, nheads, page_block_size, headdim] and match")
    if k_cache.shape[3] != hd or heads % k_cache.shape[1]:
        raise ValueError("cpu_attention: q and the caches disagree on heads or head_dim")
    if k_cache.shape[1] != heads:
        raise NotImplementedError(_MHA_ONLY)
    if not (k_cache.is_contiguous() and v_cache.is_contiguous()):
        raise ValueError("cpu_attention: the paged caches must be contiguous")
    if q.dtype not in K.DTYPES or k_cache.dtype != q.dtype or v_cache.dtype != q.dtype:
        raise ValueError("cpu_attention: q and the caches must share a dtype (fp32 or bf16)")
    if hd not in K.HEAD_DIMS or k_cache.shape[2] % 16:
        raise ValueError(f"cpu_attention: head_dim must be 32/64/128 (got {hd}) and the "
                         f"page a multiple of 16 (got {k_cache.shape[2]})")
    if page_table.dtype != torch.int32 or page_table.dim() != 2 or page_table.shape[0] != batch:
        raise ValueError("cpu_attention: page_table must be int32 [batch, max_blocks]")
    if lens.dtype != torch.int32 or lens.shape != (batch,):
        raise ValueError("cpu_attention: cache_seqlens must be an int or an int32 [batch] tensor")
    one_new = (batch, 1, heads, hd)
    if (k is None) != (v is None) or k is not None and (
            k.shape != one_new or v.shape != k.shape or k.dtype != q.dtype or v.dtype != q.dtype):
        raise ValueError("cpu_attention: k/v must both be [batch, seqlen_new, nheads, headdim]")
    if batch and int(lens.max()) + (k is not None) > page_table.shape[1] * k_cache.shape[2]:
        raise ValueError("cpu_attention: cache_seqlens exceed the page table's capacity")
    dev = q.device
    on_dev = q.is_cuda and k_cache.device == dev and v_cache.device == dev
    if not on_dev or (k is not None and (k.device != dev or v.device != dev)):
        raise ValueError(_DEVICE)
    if not (K.aligned(k_cache) and K.aligned(v_cache)):
        raise ValueError("cpu_attention: the paged caches must start 16-byte aligned")
    if k is not None:
        # k and v must share one layout with packed heads and 16-byte alignment
        if not (_heads_contiguous(k) is k and v.stride() == k.stride() and K.aligned(v)):
            k, v = k.contiguous(), v.contiguous()
        if not (K.aligned(k) and K.aligned(v)):
            k, v = (x.clone(memory_format=torch.contiguous_format) for x in (k, v))
    return _heads_contiguous(q), k_cache, v_cache, k, v, page_table.contiguous(), lens.contiguous()


def flash_attn_func(q, k, v, softmax_scale=None, causal=False):
    """Attention of every query of a sequence over every key of it: flash-attn's
    ``flash_attn_func``, forward only.

    ``q`` is ``[batch, seqlen_q, nheads, headdim]`` and ``k``/``v``
    ``[batch, seqlen_k, nheads, headdim]`` with the same head count (grouped or
    multi-query heads raise ``NotImplementedError``); any strides with a packed
    head dim are read in place, so slices of a fused QKV projection need no copy.
    ``causal`` aligns the mask to the bottom right: query ``i`` sees keys
    ``j <= i + seqlen_k - seqlen_q``, and a query that sees no key gets an output
    of zeros.  ``softmax_scale`` is the fourth positional argument (there is no
    dropout) and defaults to ``headdim ** -0.5``.
    """
    out = _flash(q, k, v, softmax_scale, causal)
    if out is None:
        q, k, v = _check_flash(q, k, v)
        out = _flash(q, k, v, softmax_scale, bool(causal))
        if out is None:
            raise RuntimeError("cpu_attention: the kernel declined arguments that passed validation")
    return out


def _flash(q, k, v, softmax_scale, causal):
    rt, _, flash = _ENTRIES or _entries()
    out = flash(rt, q, k, v, softmax_scale, causal, 0, 0)
    if type(out) is int:
        # A call whose keys are split over blocks asked for scratch (an int = the bytes it
        # needs).  It is allocated for this call on the current stream: the
        # caching allocator hands the bytes to nothing else until the kernels
        # queued on that stream have used them, and under graph capture the
        # graph's own pool keeps them for every replay.
        ws = torch.empty(out, dtype=torch.uint8, device=q.device)
        out = flash(rt, q, k, v, softmax_scale, causal, ws.data_ptr(), ws.numel())
    return out


def _check_flash(q, k, v):
    """Called once the kernel module declined a prefill: raises the error that
    names the broken rule, or returns q/k/v with a packed head dim and 16-byte
    aligned pointers and strides."""
    q, k, v = map(_as_plain, (q, k, v))
    if q.dim() != 4 or k.dim() != 4 or v.shape != k.shape:
        raise ValueError("cpu_attention: q/k/v must be [batch, seqlen, nheads, headdim]")
    batch, seq_q, heads, hd = q.shape
    if (k.shape[0] != batch or k.shape[3] != hd or heads % k.shape[2]
            or seq_q < 1 or k.shape[1] < 1):
        raise ValueError("cpu_attention: k/v must be [batch, seqlen_k, nheads, headdim] matching q")
    if k.shape[2] != heads:
        raise NotImplementedError(_MHA_ONLY)
    if q.dtype not in K.DTYPES or k.dtype != q.dtype or v.dtype != q.dtype:
        raise ValueError("cpu_attention: q/k/v must share a dtype (fp32 or bf16)")
    if hd not in K.HEAD_DIMS:
        raise ValueError(f"cpu_attention: head_dim must be 32, 64 or 128 (got {hd})")
    if not (q.is_cuda and k.device == q.device and v.device == q.device):
        raise ValueError(_DEVICE)
    readable = []
    for x in (q, k, v):
        if x.stride(3) != 1:
            x = x.contiguous()
        readable.append(_in_place_or_copy(x, [x.stride(i) if x.shape[i] > 1 else 0 for i in range(3)]))
    return readable


def flash_attn_varlen_func(q, k, v, cu_seqlens_q, cu_seqlens_k, max_seqlen_q,
                           max_seqlen_k, softmax_scale=None, causal=False):
    """Not provided: pad the sequences for ``flash_attn_func``, or keep them in the
    paged cache."""
    raise NotImplementedError("cpu_attention: variable-length attention is not ported")


def flash_attn_qkvpacked_func(qkv, *args, **kwargs):
    """Not provided: slice q, k and v out of the packed tensor and call
    ``flash_attn_func``, which reads such views in place."""
    raise NotImplementedError("cpu_attention: packed attention is not ported")


flash_attn_kvpacked_func = flash_attn_varlen_qkvpacked_func = \
    flash_attn_varlen_kvpacked_func = flash_attn_qkvpacked_func
