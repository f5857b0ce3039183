"""PyTorch-CPU restatement of the top-k decode step (TEST INFRASTRUCTURE ONLY).

The reference has no CPU decode path (every kernel launcher requires CUDA
tensors, e.g. kv_cache.py:234), so the CPU baseline of the benchmark is this
restatement of the same step, in float32 on the host's cores:

  criticality   sum_d max(q_d kmin_pd, q_d kmax_pd), the last page excluded
                (kernels/page_criticality.py:61-104, attention_topk.py:45-51)
  selection     torch.topk of k = min(budget // ps, P - 1) pages per head,
                ascending, the last page appended (attention_topk.py:52-71,
                kv_cache.py:167-185)
  decode        the selected K rows gathered, s = (alpha-1)/sqrt(D) q.k, the
                exact entmax threshold by the sort-based closed form (alpha 2:
                sparsemax; alpha 1.5: Peters et al. 2019), out = sum p v
                (kernels/adadecode_paged.py:567-762 once its tau has converged)

MHA only (H == Hkv), no ALiBi: the benchmark's headline shape.  Only
``bench.py``'s cpu_baseline leg and ``tests/`` use this module; it is never
on the product path.  Pinned by tests/test_oracle.py against the NumPy oracle's
topk_decode_step (converged tau).
"""

from __future__ import annotations

import math

import torch


def entmax_tau_sorted(s: torch.Tensor, alpha: float) -> torch.Tensor:
    """Exact threshold of every row of ``s`` [..., n] (already (alpha-1)-scaled)."""
    z, _ = torch.sort(s, dim=-1, descending=True)
    n = z.shape[-1]
    k = torch.arange(1, n + 1, dtype=s.dtype, device=s.device)
    cs = torch.cumsum(z, dim=-1)
    if alpha == 2.0:
        supp = 1.0 + k * z > cs
        kk = supp.to(torch.int64).cumsum(-1).amax(-1, keepdim=True)  # support is a prefix
        return ((cs.gather(-1, kk - 1) - 1.0) / kk.to(s.dtype)).squeeze(-1)
    if alpha == 1.5:
        mean = cs / k
        meansq = torch.cumsum(z * z, dim=-1) / k
        delta = (1.0 - k * (meansq - mean * mean)) / k
        tau = mean - torch.sqrt(torch.clamp(delta, min=0.0))
        supp = tau <= z
        kk = supp.to(torch.int64).cumsum(-1).amax(-1, keepdim=True)
        return tau.gather(-1, kk - 1).squeeze(-1)
    raise ValueError("alpha must be 1.5 or 2")


def topk_decode_step(q, k_cache, v_cache, k_min, k_max, token_budget: int, page_size: int,
                     alpha: float) -> torch.Tensor:
    """One top-k decode step on the CPU.

    q [B, H, D]; k_cache, v_cache [B, H, S, D] (any float dtype, gathered rows
    are converted to float32); k_min, k_max [B, H, P, D].  Returns out [B, H, D]
    float32.
    """
    B, H, D = q.shape
    S = k_cache.shape[2]
    ps = page_size
    P = (S + ps - 1) // ps
    n_sel = min(token_budget // ps, P - 1)
    qf = q.float()
    bound = torch.where(qf[:, :, None, :] >= 0, k_max[:, :, :P - 1].float(),
                        k_min[:, :, :P - 1].float())
    scores = torch.einsum("bhpd,bhd->bhp", bound, qf)
    sel = torch.topk(scores, n_sel, dim=-1).indices.sort(dim=-1).values
    last = torch.full((B, H, 1), P - 1, dtype=sel.dtype)
    pages = torch.cat([sel, last], dim=-1)
    rows = (pages[..., None] * ps + torch.arange(ps)).reshape(B, H, -1)
    n_tok = n_sel * ps + (S - (P - 1) * ps)
    rows = rows[..., :n_tok]
    idx = rows[..., None].expand(B, H, n_tok, D)
    kr = torch.gather(k_cache, 2, idx).float()
    vr = torch.gather(v_cache, 2, idx).float()
    s = torch.einsum("bhnd,bhd->bhn", kr, qf) * ((alpha - 1.0) / math.sqrt(D))
    tau = entmax_tau_sorted(s, alpha)
    p = torch.clamp(s - tau[..., None], min=0.0)
    if alpha == 1.5:
        p = p * p
    return torch.einsum("bhn,bhnd->bhd", p, vr)
