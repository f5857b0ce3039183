"""Row-wise alpha-entmax with autograd (mirrors entmaxkv/kernels/triton_entmax.py).

``triton_entmax``, ``triton_sparsemax`` and ``triton_entmax15`` keep the
reference names and signatures (kernels/triton_entmax.py:686-723) and run the
HIP kernels of ``ekv_entmax_rows_forward`` / ``ekv_entmax_rows_backward``.

One difference a caller can see: the reference stops after ``n_iter`` hybrid
Halley/secant steps from a histogram initialisation (:441-511), so its rows
sum to 1 only approximately; here tau is solved exactly (alpha 2 and 1.5: the
closed-form root on the refined support; other alpha: bracketed Halley to fp32
resolution).  ``n_iter``, ``use_histogram`` and ``fast_math`` are accepted and
do not change results.
"""

from __future__ import annotations

import torch

from ._lib import call, dtype_code, ptr, require_gpu, stream_ptr


def _rows(t: torch.Tensor) -> torch.Tensor:
    """[rows, n] view with a unit last stride (copied when that is not possible)."""
    t2 = t.reshape(-1, t.shape[-1]) if t.dim() != 2 else t
    return t2 if t2.stride(-1) == 1 else t2.contiguous()


def entmax_forward(x: torch.Tensor, alpha: float = 1.5,
                   tau_out: torch.Tensor | None = None) -> torch.Tensor:
    """alpha-entmax over the last dim of x; ``tau_out`` ([rows] float32) receives
    the threshold on the (alpha - 1) x scale."""
    require_gpu(x)
    if not alpha > 1.0:
        raise ValueError(f"alpha must be > 1 (got {alpha})")
    if x.shape[-1] == 0:
        return torch.empty_like(x)
    x2 = _rows(x)
    y = torch.empty(x.shape, dtype=x.dtype, device=x.device)
    y2 = y.view(-1, x.shape[-1])
    if tau_out is not None:
        assert tau_out.dtype == torch.float32 and tau_out.is_contiguous() \
            and tau_out.numel() == x2.shape[0], "tau_out must be contiguous float32 [rows]"
    call("ekv_entmax_rows_forward", x2.data_ptr(), x2.stride(0), y2.data_ptr(), y2.stride(0),
         x2.shape[0], x2.shape[1], float(alpha), ptr(tau_out), dtype_code(x.dtype),
         stream_ptr(x.device))
    return y


def entmax_backward(y: torch.Tensor, dy: torch.Tensor, alpha: float) -> torch.Tensor:
    """Gradient of alpha-entmax at output y (kernels/triton_entmax.py:536-612)."""
    require_gpu(y, dy)
    if dy.dtype != y.dtype:
        dy = dy.to(y.dtype)
    if y.shape[-1] == 0:
        return torch.empty_like(y)
    y2 = _rows(y)
    g2 = _rows(dy)
    dx = torch.empty(y.shape, dtype=y.dtype, device=y.device)
    d2 = dx.view(-1, y.shape[-1])
    call("ekv_entmax_rows_backward", y2.data_ptr(), y2.stride(0), g2.data_ptr(), g2.stride(0),
         d2.data_ptr(), d2.stride(0), y2.shape[0], y2.shape[1], float(alpha),
         dtype_code(y.dtype), stream_ptr(y.device))
    return dx


class _entmax_native(torch.autograd.Function):
    """Autograd wrapper (kernels/triton_entmax.py:616-683)."""

    @staticmethod
    def forward(ctx, x, alpha=1.5, n_iter=10, use_histogram=True, fast_math=False):
        y = entmax_forward(x, alpha)
        ctx.save_for_backward(y)
        ctx.alpha = alpha
        return y

    @staticmethod
    def backward(ctx, dy):
        (y,) = ctx.saved_tensors
        return entmax_backward(y, dy, ctx.alpha), None, None, None, None


def triton_entmax(x: torch.Tensor, alpha: float = 1.5, n_iter: int = 2,
                  use_histogram: bool = True, fast_math: bool = False) -> torch.Tensor:
    """alpha-entmax over the last dim (kernels/triton_entmax.py:686-713)."""
    return _entmax_native.apply(x, alpha, n_iter, use_histogram, fast_math)


def triton_sparsemax(x: torch.Tensor, **kwargs) -> torch.Tensor:
    """Sparsemax, entmax with alpha = 2 (kernels/triton_entmax.py:716-718)."""
    return triton_entmax(x, alpha=2.0, **kwargs)


def triton_entmax15(x: torch.Tensor, **kwargs) -> torch.Tensor:
    """1.5-entmax (kernels/triton_entmax.py:721-723)."""
    return triton_entmax(x, alpha=1.5, **kwargs)
