"""Top-k page selection feeding the paged entmax decode (mirrors entmaxkv/attention_topk.py)."""

from __future__ import annotations

import torch

from . import kernels as K
from .kv_cache import PagedKVCache


def sparse_attention_decode_paged(
    q: torch.Tensor,
    kv_cache: PagedKVCache,
    k_new: torch.Tensor,
    v_new: torch.Tensor,
    out: torch.Tensor,
    token_budget: int,
    cache_seqlens: torch.Tensor,
    q_seqlens: torch.Tensor,
    alibi_slopes: torch.Tensor = None,
    alpha: float = 1.5,
    splits: int = 32,
    niter: int = 10,
    append_cache: bool = True,
    use_triton_criticality: bool = True,
    workspace=None,
):
    """Decode-phase attention with top-k page selection (attention_topk.py:8-100).

    Launches: [append] -> criticality + top-k (one kernel) -> scores + tau ->
    weighted sum.  ``cache_seqlens`` is the compacted token count supplied by the
    caller, as in the reference (n_selected * page_size + last_page_size).
    ``splits`` and ``use_triton_criticality`` are accepted for compatibility.
    Under GQA the page table is per kv head (group maximum of page scores).
    """
    batch, num_heads, _, head_dim = q.shape
    num_kv_heads = kv_cache.k_cache.shape[1]

    if append_cache:
        kv_cache.append(k_new, v_new)

    seq_len = kv_cache.seq_len
    page_size = kv_cache.page_size
    total_pages = (seq_len + page_size - 1) // page_size
    num_pages_to_select = min(token_budget // page_size, total_pages - 1)

    page_indices = kv_cache.select_topk(q, num_pages_to_select, alibi_slopes=alibi_slopes)

    if workspace is None:
        workspace = kv_cache.get_paged_decode_workspace(
            batch, num_heads, head_dim, splits, 16, q.dtype, q.device,
            max_tokens=(num_pages_to_select + 1) * page_size)

    K.paged_entmax_decode(
        q, kv_cache._k, kv_cache._v, out, cache_seqlens, page_indices, page_size, alpha,
        tau_mode=0, iters=niter, tau=None, alibi_slopes=alibi_slopes, q_seqlens=q_seqlens,
        workspace=workspace, kv_rows=kv_cache.kv_capacity)
    return out
