"""Gaussian-aware page selection feeding the paged entmax decode
(mirrors entmaxkv/attention_gaussian.py)."""

from __future__ import annotations

import math
from typing import Optional

import torch

from . import kernels as K
from .gaussian_utils import solve_for_tau_hat_page_gaussian_mixture_auto, stats_dict
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
    A ragged cache (``kv_cache.seq_lens``) gives every sequence its own pages,
    statistics and tau-hat; the automatic margins stay batch-wide.
    Launches: [append] -> page moments -> [page-mixture tau-hat under ALiBi]
    -> one launch of global moments + tau-hat + select + pack + clamp +
    decode (separate launches when batch * kv heads is too small to fill the
    GPU).
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

    last_page_tokens = seq_len - (num_pages - 1) * page_size if num_pages > 1 else 0
    seq_len_for_stats = seq_len - last_page_tokens
    if alpha not in (2, 1.5, 4 / 3):
        raise ValueError(f"Unsupported alpha for the Gaussian tau solve: {alpha}")
    buf = kv_cache.get_gaussian_buffers(q, pages_for_stats)
    seq_lens = kv_cache.seq_lens
    if q_seqlens is None and seq_lens is not None:
        q_seqlens = seq_lens
    K.compute_page_gaussian_moments(q, kv_cache.k_mean, kv_cache.k_std, pages_for_stats, buf,
                                    alibi_slopes=alibi_slopes, page_size=page_size,
                                    seq_len=seq_len, n_tokens=seq_len_for_stats,
                                    seq_lens=seq_lens)
    tau_hat_given = alibi_slopes is not None
    if tau_hat_given:
        # ALiBi: page-mixture tau-hat over the biased page means (gaussian_utils.py:171-181)
        tau_mix = solve_for_tau_hat_page_gaussian_mixture_auto(
            buf.mu_p, buf.sigma_p, alpha=alpha, uniform_page_count=float(page_size),
            seq_lens=seq_lens, page_size=page_size)
        buf.tau_hat.copy_(tau_mix.squeeze(-1))
    gaussian_stats = stats_dict(buf, seq_len_for_stats, pages_for_stats, num_pages,
                                threshold_excess_margin_fraction, tau_clamp_page_max_quantile)

    last_page_size = (seq_len - (math.ceil(seq_len / page_size) - 1) * page_size
                      if seq_len > page_size else seq_len)
    do_clamp = needs_tau and clamp_tau
    sb = kv_cache._get_select_buffers(batch, num_heads, kv_cache.num_kv_heads, num_pages,
                                      q.device)
    workspace = kv_cache.get_paged_decode_workspace(
        batch, num_heads, head_dim, splits, 16, q.dtype, q.device,
        max_tokens=num_pages * page_size)
    if tau_mode == "exact":
        dec_mode, iters = 0, niter
    else:
        dec_mode = 1
        if tau_correction_iters is None:
            if tau_mode == "fixed":
                tau_correction_iters = 0
            else:
                tau_correction_iters = 1 if alibi_slopes is None else 2
        iters = tau_correction_iters
    kc, vc, rows, blocks = kv_cache.kv_operands()
    K.gaussian_paged_entmax_decode(
        q, kc, vc, out, buf, pages_for_stats=pages_for_stats,
        num_pages=num_pages, n_tokens=seq_len_for_stats, page_size=page_size, alpha=alpha,
        tau_hat_given=tau_hat_given, safety_margin_z=None, max_quantile=None,
        threshold_excess_margin_fraction=threshold_excess_margin_fraction,
        page_indices=sb["page_indices"], counts=sb["counts"], tau_floor=sb["tau_floor"],
        cache_seqlens=sb["cache_seqlens"], last_page_size=last_page_size,
        tau_clamped=sb["tau_clamped"] if do_clamp else None,
        clamp_quantile=tau_clamp_page_max_quantile, effective=sb["effective"],
        tau_out=workspace.taus, tau_mode=dec_mode, iters=iters, workspace=workspace,
        alibi_slopes=alibi_slopes, q_seqlens=q_seqlens, kv_rows=rows,
        seq_lens=seq_lens, blocks=blocks)
    kv_cache.record_gaussian_selection(gaussian_stats, sb, do_clamp)
    if tau_mode != "exact":
        gaussian_stats["tau_final"] = workspace.taus
    kv_cache.last_gaussian_stats = gaussian_stats
    return out
