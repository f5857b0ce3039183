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

    Launches: [append] -> one kernel per (b, kv head) that scores every page,
    selects the top-k pages and runs the exact-tau decode on them (two kernels
    when a head does not fit one workgroup's LDS or the batch is small).  ``cache_seqlens`` is the compacted token count supplied by the
    caller, as in the reference (n_selected * page_size + last_page_size).
    ``splits`` and ``use_triton_criticality`` are accepted for compatibility.
    Under GQA the page table is per kv head: the k pages of best rank over the
    group's query heads (round robin over each head's own page order).
    Ragged cache (``kv_cache.seq_lens``): each sequence selects
    min(budget // ps, P_b - 1) pages of its own; ``cache_seqlens`` may then be
    None (derived per sequence, ``PagedKVCache.compacted_seqlens``) and
    ``q_seqlens`` defaults to the sequence lengths.
    """
    batch, num_heads, _, head_dim = q.shape
    num_kv_heads = kv_cache.num_kv_heads

    # a uniform batch's new row is written by the step's own launch
    row = None
    if append_cache:
        if kv_cache.is_ragged or k_new.shape[2] != 1:
            kv_cache.append(k_new, v_new)
        else:
            row = kv_cache.reserve_append(k_new, v_new)

    seq_len = kv_cache.seq_len
    page_size = kv_cache.page_size
    seq_lens = kv_cache.seq_lens
    if cache_seqlens is None:
        cache_seqlens = kv_cache.compacted_seqlens(token_budget)
    if q_seqlens is None and seq_lens is not None:
        q_seqlens = seq_lens
    total_pages = (seq_len + page_size - 1) // page_size
    num_pages_to_select = min(token_budget // page_size, total_pages - 1)

    if workspace is None:
        workspace = kv_cache.get_paged_decode_workspace(
            batch, num_heads, head_dim, splits, 16, q.dtype, q.device,
            max_tokens=(num_pages_to_select + 1) * page_size)

    if num_pages_to_select == 0:
        if row is not None:
            kv_cache.write_append(row)
        page_indices = kv_cache.select_topk(q, 0, alibi_slopes=alibi_slopes)
        kc, vc, rows, blocks = kv_cache.kv_operands()
        K.paged_entmax_decode(
            q, kc, vc, out, cache_seqlens, page_indices, page_size, alpha,
            tau_mode=0, iters=niter, tau=None, alibi_slopes=alibi_slopes, q_seqlens=q_seqlens,
            workspace=workspace, kv_rows=rows, blocks=blocks)
        return out

    # criticality + top-k + decode in one launch (two when the shape needs it)
    last = total_pages - 1
    page_indices = kv_cache.get_page_indices_buf(batch, num_kv_heads, num_pages_to_select, last)
    scores = kv_cache._get_scores_buf(batch, num_heads, total_pages - 1, q.dtype, q.device)
    kv_cache.last_page_scores = scores
    kc, vc, rows, blocks = kv_cache.kv_operands()
    K.topk_paged_entmax_decode(
        q, kv_cache.k_min, kv_cache.k_max, scores, num_pages_to_select, last, kc,
        vc, out, page_indices, cache_seqlens, page_size, alpha, niter, seq_len,
        seq_len - 1, alibi_slopes=alibi_slopes, q_seqlens=q_seqlens, workspace=workspace,
        kv_rows=rows, seq_lens=seq_lens, blocks=blocks, append=row)
    return out
