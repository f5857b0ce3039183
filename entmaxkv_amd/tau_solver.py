"""Single-Gaussian tau-hat (mirrors entmaxkv/tau_solver.py:347-412).

The reference dispatches to a Triton kernel on CUDA tensors and to Python
scalar loops otherwise; this module always runs the native kernel and rejects
CPU tensors.
"""

from __future__ import annotations

import torch

from . import kernels as K


def solve_for_tau_hat_single_gaussian(mu_g: torch.Tensor, sigma_g: torch.Tensor, n: int,
                                      alpha: float, max_iter: int = 120, tol: float = 1e-6,
                                      verbose: bool = False) -> torch.Tensor:
    """Root tau of n*E[[(alpha-1)S - tau]_+^(1/(alpha-1))] = 1, S ~ N(mu_g, sigma_g^2)."""
    if alpha not in (2, 1.5, 4 / 3):
        raise ValueError(f"Unsupported alpha for the native tau solve: {alpha}")
    tau = K.solve_for_tau_hat_single_gaussian_gpu(mu_g, sigma_g, n, alpha, iterations=max_iter,
                                                  tol=tol)
    return tau.to(dtype=mu_g.dtype)
