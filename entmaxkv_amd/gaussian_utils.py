"""Gaussian score statistics and tau clamping (mirrors entmaxkv/gaussian_utils.py).

Differences from the reference, all on the host side:
* the automatic ``safety_margin_z``/``max_quantile`` (gaussian_utils.py:163-169)
  are derived on the device inside the selection launch, so no ``.item()``
  synchronisation happens per decode step; the dict carries None for them;
* tau-hat is solved on the device right after the global moments (single
  Gaussian, one wave per head) or by one extra launch (page mixture, ALiBi
  only).
"""

from __future__ import annotations

import math
from typing import Optional

import torch

from . import kernels as K


def solve_for_tau_hat_page_gaussian_mixture_auto(mu_pages, sigma_pages, page_counts=None,
                                                 alpha: float = 1.5, max_iter: int = 40,
                                                 tol: float = 1e-6,
                                                 uniform_page_count: float = 1.0,
                                                 seq_lens=None, page_size: int = 16):
    """gaussian_utils.py:16-49 (always the native kernel).  With ``seq_lens`` (a
    ragged batch, rows [B, H, ...]) row (b, h) mixes only sequence b's pages."""
    return K.solve_for_tau_hat_page_gaussian_mixture(
        mu_pages, sigma_pages, page_counts=page_counts, alpha=alpha, max_iter=max_iter, tol=tol,
        uniform_page_count=uniform_page_count, seq_lens=seq_lens, page_size=page_size)


def compute_gaussian_aware_statistics(q, k_mean, k_std, seq_len: int, page_size: int,
                                      alpha: float = 1.5, alibi_slopes=None,
                                      use_triton_stats: bool = True,
                                      threshold_excess_margin_fraction: float = 0.2,
                                      tau_clamp_page_max_quantile: float = 0.50,
                                      safety_margin_z: Optional[float] = None,
                                      max_quantile: Optional[float] = None,
                                      buffers: Optional[K.GaussianBuffers] = None):
    """Gaussian score statistics and tau-hat (gaussian_utils.py:66-200).

    Returns the reference's stats dict; ``tau_hat`` is [B, H] float32.
    ``use_triton_stats`` is accepted for compatibility (the native kernel always runs).
    """
    num_pages = k_mean.shape[2]
    pages_for_stats = num_pages - 1 if num_pages > 1 else num_pages
    last_page_tokens = seq_len - (num_pages - 1) * page_size if num_pages > 1 else 0
    seq_len_for_stats = seq_len - last_page_tokens
    if alpha not in (2, 1.5, 4 / 3):
        raise ValueError(f"Unsupported alpha for the Gaussian tau solve: {alpha}")
    use_mixture = alibi_slopes is not None
    buf = K.compute_page_gaussian_stats(
        q, k_mean, k_std, pages_for_stats, alibi_slopes=alibi_slopes, page_size=page_size,
        seq_len=seq_len, alpha=alpha, n_tokens=seq_len_for_stats, solve_tau=not use_mixture,
        buffers=buffers)
    if use_mixture:
        tau_hat = solve_for_tau_hat_page_gaussian_mixture_auto(
            buf.mu_p, buf.sigma_p, alpha=alpha, uniform_page_count=float(page_size))
        buf.tau_hat.copy_(tau_hat.squeeze(-1))
    return stats_dict(buf, seq_len_for_stats, pages_for_stats, num_pages,
                      threshold_excess_margin_fraction, tau_clamp_page_max_quantile,
                      safety_margin_z, max_quantile)


def stats_dict(buf, seq_len_for_stats: int, pages_for_stats: int, num_pages: int,
               threshold_excess_margin_fraction: float, tau_clamp_page_max_quantile: float,
               safety_margin_z=None, max_quantile=None) -> dict:
    """The reference's statistics dict (gaussian_utils.py:183-200) over the
    device buffers of one step."""
    return {
        "mu_scores_per_page": buf.mu_p,
        "sigma_scores_per_page": buf.sigma_p,
        "mu_global": buf.mu_g,
        "sigma_global": buf.sigma_g,
        "tau_hat": buf.tau_hat,
        "seq_len_for_stats": seq_len_for_stats,
        "pages_for_stats": pages_for_stats,
        "num_pages": num_pages,
        "safety_margin_z": safety_margin_z,
        "threshold_excess_margin_fraction": threshold_excess_margin_fraction,
        "tau_clamp_page_max_quantile": tau_clamp_page_max_quantile,
        "max_quantile": max_quantile,
        "mean_variance": buf.mean_var,
        "variance_of_means": buf.var_means,
    }


def clamp_tau_to_selected_page_statistics(tau, gaussian_stats: dict, page_indices,
                                          num_selected_per_head, page_size: int, alpha: float,
                                          eps: float = 1.0e-4):
    """Clamp tau to the selected pages' score caps (gaussian_utils.py:203-315)."""
    if tau is None:
        return tau
    return K.clamp_tau_to_selected_page_statistics(
        tau, gaussian_stats["mu_scores_per_page"], gaussian_stats["sigma_scores_per_page"],
        page_indices, num_selected_per_head, gaussian_stats.get("tau_floor"), page_size, alpha,
        gaussian_stats.get("tau_clamp_page_max_quantile", 0.50),
        gaussian_stats["pages_for_stats"], eps=eps)
