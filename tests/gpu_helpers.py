"""Shared helpers for the GPU parity tests (inputs are generated on the CPU so
the oracle and the HIP path see identical bits)."""

from __future__ import annotations

import numpy as np
import torch

from oracle import entmaxkv_oracle as O

TORCH_DT = {"fp16": torch.float16, "bf16": torch.bfloat16, "fp32": torch.float32}

# Output tolerance: max-abs 2e-3 for fp16/bf16 and 1e-5 for fp32 on the value
# before the final store, plus one unit in the last place of the output dtype
# for the store's rounding (the kernel rounds its fp32 result once).
ATOL = {"fp16": 2e-3, "bf16": 2e-3, "fp32": 1e-5}
ULP = {"fp16": 2.0 ** -10, "bf16": 2.0 ** -7, "fp32": 2.0 ** -23}


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
