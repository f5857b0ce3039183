"""Shared helpers for the GPU parity tests (inputs are generated on the CPU so
the oracle and the HIP path see identical bits)."""

from __future__ import annotations

import numpy as np
import torch

from oracle import entmaxkv_oracle as O

TORCH_DT = {"fp16": torch.float16, "bf16": torch.bfloat16, "fp32": torch.float32}

# Output tolerance: max-abs 2e-3 for fp16/bf16 and 1e-5 for fp32 on every
# output.  bf16 alone adds half a unit in the last place of |ref| (2^-8 |ref|):
# with 8 significant bits, storing an output above 0.52 in magnitude rounds it
# by more than 2e-3 by itself, in the reference's stored output as much as in
# this one.  fp16 (11 bits) rounds an output below 4 by at most 2^-11 * 4 =
# 9.8e-4 and fp32 by far less, so they take no such term.
ATOL = {"fp16": 2e-3, "bf16": 2e-3, "fp32": 1e-5}
ULP = {"fp16": 0.0, "bf16": 2.0 ** -8, "fp32": 0.0}


def randn(rng, shape, dtype, scale=1.0):
    x = rng.standard_normal(shape) * scale
    return O.round_to(x, dtype)


def to_dev(x, dtype, device="cuda"):
    return torch.tensor(np.asarray(x, dtype=np.float64), dtype=torch.float64).to(TORCH_DT[dtype]).to(device)


def to_np(t):
    return t.detach().to(torch.float64).cpu().numpy()


def assert_out_close(got, ref, dtype, what="out"):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    tol = ATOL[dtype] + ULP[dtype] * np.abs(ref)
    err = np.abs(got - ref)
    bad = err > tol
    assert not bad.any(), (f"{what}: {bad.sum()} of {bad.size} beyond tolerance; "
                           f"max err {err.max():.3g} (dtype {dtype})")


def ulp_diff_16(a, b, dtype):
    """Distance in units of the dtype's ulp at |b| (for stats / score checks)."""
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    mant = {"fp16": 10, "bf16": 7, "fp32": 23}[dtype]
    e = np.floor(np.log2(np.maximum(np.abs(b), 2.0 ** -14)))
    return np.abs(a - b) / 2.0 ** (e - mant)


def gqa_structured_case(rng, B, Hkv, G, S, D, ps, dtype, n_own, n_shared, beta):
    """GQA inputs where the group's query heads want different pages: per kv
    head, n_shared pages pulled toward the group's mean query direction and
    n_own pages per query head pulled toward that head's direction (keys +=
    beta * direction); query norms differ per head (x0.5..2).  Returns float64
    arrays q [B, H, D], k, v [B, Hkv, S, D] already rounded to ``dtype``."""
    H = Hkv * G
    P = S // ps
    q = rng.standard_normal((B, H, D)) * rng.uniform(0.5, 2.0, (1, H, 1))
    k = rng.standard_normal((B, Hkv, S, D))
    v = rng.standard_normal((B, Hkv, S, D))
    for b in range(B):
        for kvh in range(Hkv):
            pages = rng.choice(P - 1, n_shared + G * n_own, replace=False)
            qh = [q[b, kvh * G + g] / np.linalg.norm(q[b, kvh * G + g]) for g in range(G)]
            mean = sum(qh) / np.linalg.norm(sum(qh))
            for i, p in enumerate(pages):
                d = mean if i < n_shared else qh[(i - n_shared) // n_own]
                k[b, kvh, p * ps:(p + 1) * ps] += beta * d
    return O.round_to(q, dtype), O.round_to(k, dtype), O.round_to(v, dtype)


def dense_entmax_attention(q, K, V, alpha, dtype):
    """Exact entmax attention of every query head over all of its kv head's
    keys (float64): the accuracy reference of the sparse decode steps."""
    B, H, D = q.shape
    G = H // K.shape[1]
    qs = O.scaled_query(q, alpha, dtype)
    out = np.zeros((B, H, D))
    for b in range(B):
        for h in range(H):
            s = np.asarray(K[b, h // G], np.float64) @ qs[b, h]
            out[b, h] = O.entmax_exact(s, alpha) @ np.asarray(V[b, h // G], np.float64)
    return out


def rel_error(out, ref):
    """||out - ref|| / ||ref|| over the whole tensor (tests/benchmark_utils.py:38-49)."""
    return float(np.linalg.norm(np.asarray(out) - ref) / np.linalg.norm(ref))
