"""EntmaxKV sparse-entmax paged decode for AMD Instinct MI355X (gfx950).

Drop-in for the public API of deep-spin/entmaxkv (entmaxkv/__init__.py:1-15):
``PagedKVCache``, ``sparse_attention_decode_paged`` and
``sparse_attention_decode_gaussian_aware_entmax``, backed by hand-written HIP
kernels in ``libentmaxkv_hip.so`` (C ABI: include/entmaxkv.h).
"""

from .kv_cache import PagedKVCache
from .attention_topk import sparse_attention_decode_paged
from .attention_gaussian import sparse_attention_decode_gaussian_aware_entmax

__all__ = [
    "PagedKVCache",
    "sparse_attention_decode_paged",
    "sparse_attention_decode_gaussian_aware_entmax",
]
