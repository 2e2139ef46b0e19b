# Derived from ducviet00/cpu-attention (cpu_attention/__init__.py), Apache
# License 2.0; modified for the MI355X build (see NOTICE at the repository root).
# The export list is the original package's, so that imports keep working.

"""The three attention ops of ducviet00/cpu-attention, computed on an AMD Instinct
MI355X (gfx950) by hand-written CDNA4 kernels behind a C ABI
(``libcpu_attention_hip.so``), with the original package's flash-attn-style
functions, arguments, errors and cache layout.

The KV cache is head-major, ``[num_blocks, nheads_k, page_block_size, headdim]``
with K transposed inside each page -- not flash-attn's page-major layout -- so
``reshape_and_cache`` (vLLM's signature) is exported to fill it.
"""

from .cache import reshape_and_cache
from .flash_attn_interface import (
    flash_attn_func,
    flash_attn_kvpacked_func,
    flash_attn_qkvpacked_func,
    flash_attn_varlen_func,
    flash_attn_varlen_kvpacked_func,
    flash_attn_varlen_qkvpacked_func,
    flash_attn_with_kvcache,
)

__version__ = "0.1.0"

__all__ = [
    "__version__",
    "flash_attn_func",
    "flash_attn_kvpacked_func",
    "flash_attn_qkvpacked_func",
    "flash_attn_varlen_func",
    "flash_attn_varlen_kvpacked_func",
    "flash_attn_varlen_qkvpacked_func",
    "flash_attn_with_kvcache",
    "reshape_and_cache",
]
