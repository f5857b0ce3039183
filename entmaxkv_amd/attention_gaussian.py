"""Gaussian-aware page selection feeding the paged entmax decode
(mirrors entmaxkv/attention_gaussian.py)."""

from __future__ import annotations

import math
from typing import Optional

import torch

from . import kernels as K
from .gaussian_utils import compute_gaussian_aware_statistics
from .kv_cache import PagedKVCache


def sparse_attention_decode_gaussian_aware_entmax(
    q: torch.Tensor,
    kv_cache: PagedKVCache,
    k_new: torch.Tensor,
    v_new: torch.Tensor,
    out: torch.Tensor,
    alpha: float = 1.5,
    safety_margin_z: float = 0.0,
    max_quantile: float = 0.995,
    alibi_slopes: torch.Tensor = None,
    scale: Optional[float] = None,
    splits: int = 32,
    niter: int = 2,
    append_cache: bool = False,
    tau_mode: str = "corrected",
    tau_correction_iters: Optional[int] = None,
    clamp_tau: bool = True,
    threshold_excess_margin_fraction: Optional[float] = 0.2,
    tau_clamp_page_max_quantile: float = 0.50,
    q_seqlens: torch.Tensor = None,
):
    """Gaussian-aware page selection + paged entmax (attention_gaussian.py:20-144).

    tau_mode: "exact" runs the exact tau solve over the selected pages,
    "fixed" uses the Gaussian tau-hat directly, "corrected" applies
    ``tau_correction_iters`` (default 1, 2 with ALiBi) Halley corrections.
    As in the reference, ``safety_margin_z`` and ``max_quantile`` are superseded
    by the automatic margins and ``scale`` is unused (the kernel uses 1/sqrt(D)).
    Launches: [append] -> page moments + tau-hat -> [mixture tau-hat] ->
    select + pack + clamp + lengths -> scores + tau -> weighted sum.
    """
    batch, num_heads, _, head_dim = q.shape

    if scale is None:
        scale = 1.0 / math.sqrt(head_dim)

    tau_mode = tau_mode.lower()
    if tau_mode not in ("exact", "fixed", "corrected"):
        raise ValueError(f"Unsupported tau_mode={tau_mode!r}; expected 'exact', 'fixed', or 'corrected'")
    if threshold_excess_margin_fraction is None:
        raise TypeError("threshold_excess_margin_fraction must be a float")

    if append_cache:
        kv_cache.append(k_new, v_new)

    seq_len = kv_cache.seq_len
    page_size = kv_cache.page_size
    needs_tau = tau_mode != "exact"
    num_pages = kv_cache.num_pages
    pages_for_stats = num_pages - 1 if num_pages > 1 else num_pages

    gaussian_stats = compute_gaussian_aware_statistics(
        q=q, k_mean=kv_cache.k_mean, k_std=kv_cache.k_std, seq_len=seq_len, page_size=page_size,
        alpha=alpha, alibi_slopes=alibi_slopes,
        threshold_excess_margin_fraction=threshold_excess_margin_fraction,
        tau_clamp_page_max_quantile=tau_clamp_page_max_quantile,
        buffers=kv_cache.get_gaussian_buffers(q, pages_for_stats))

    last_page_size = (seq_len - (math.ceil(seq_len / page_size) - 1) * page_size
                      if seq_len > page_size else seq_len)
    do_clamp = needs_tau and clamp_tau
    page_indices, _ = kv_cache.select_gaussian_aware(
        q, alpha=alpha, safety_margin_z=safety_margin_z, max_quantile=max_quantile,
        gaussian_stats=gaussian_stats, clamp=do_clamp, last_page_size=last_page_size)
    cache_seqlens = gaussian_stats["cache_seqlens"]

    workspace = kv_cache.get_paged_decode_workspace(
        batch, num_heads, head_dim, splits, 16, q.dtype, q.device,
        max_tokens=page_indices.shape[2] * page_size)

    if tau_mode == "exact":
        K.paged_entmax_decode(
            q, kv_cache._k, kv_cache._v, out, cache_seqlens, page_indices, page_size, alpha,
            tau_mode=0, iters=niter, tau=None, alibi_slopes=alibi_slopes, q_seqlens=q_seqlens,
            workspace=workspace, kv_rows=kv_cache.kv_capacity)
    else:
        if tau_correction_iters is None:
            if tau_mode == "fixed":
                tau_correction_iters = 0
            else:
                tau_correction_iters = 1 if alibi_slopes is None else 2
        tau0 = gaussian_stats["tau_clamped"] if do_clamp else gaussian_stats["tau_hat"]
        K.paged_entmax_decode(
            q, kv_cache._k, kv_cache._v, out, cache_seqlens, page_indices, page_size, alpha,
            tau_mode=1, iters=tau_correction_iters, tau=workspace.taus, tau_in=tau0,
            alibi_slopes=alibi_slopes, q_seqlens=q_seqlens, workspace=workspace,
            kv_rows=kv_cache.kv_capacity)
        gaussian_stats["tau_final"] = workspace.taus
    kv_cache.last_gaussian_stats = gaussian_stats
    return out
