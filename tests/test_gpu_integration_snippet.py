"""Runs the integration guide's reference-side ctypes binding on the GPU and
compares its scores with entmaxkv_amd's own criticality launcher and with the
oracle (kernels/page_criticality.py:107-187 is the interface it replaces)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import entmaxkv_oracle as O
from tests.gpu_helpers import randn, to_dev, to_np

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("dtype", ["fp16", "bf16", "fp32"])
@pytest.mark.parametrize("alibi", [False, True])
@pytest.mark.parametrize("G", [1, 4])
def test_integration_snippet_scores(dtype, alibi, G):
    from entmaxkv_amd import _lib, kernels as K
    from integration_snippet import load_snippet

    print(f"CASE snippet dtype={dtype} alibi={alibi} G={G}", flush=True)
    mod = load_snippet(_lib.LIB_PATH)
    rng = np.random.default_rng(7 + G)
    B, Hkv, D, ps, S = 2, 4, 128, 16, 16 * 40 + 5
    H = Hkv * G
    k = randn(rng, (B, Hkv, S, D), dtype)
    q = randn(rng, (B, H, 1, D), dtype)
    kmin, kmax, _, _ = O.page_stats(k, ps, dtype)
    slopes_kv = np.linspace(0.05, 0.4, Hkv)
    kw = {}
    if alibi:
        kw = dict(alibi_slopes=torch.tensor(slopes_kv, dtype=torch.float32, device="cuda"),
                  q_pos=S - 1, seq_len=S)
    tq, tmin, tmax = to_dev(q, dtype), to_dev(kmin, dtype), to_dev(kmax, dtype)
    got = mod.triton_estimate_page_criticality(tq, tmin, tmax, page_size=ps,
                                               exclude_last_page=True, **kw)
    kw2 = dict(kw)
    if alibi:  # entmaxkv_amd takes one slope per query head
        kw2["alibi_slopes"] = kw["alibi_slopes"].repeat_interleave(G)
    mine = K.estimate_page_criticality(tq, tmin, tmax, page_size=ps, exclude_last_page=True,
                                       **kw2)
    torch.cuda.synchronize()
    assert got.shape == (B, H, kmin.shape[2] - 1) and got.dtype == tq.dtype
    np.testing.assert_array_equal(to_np(got), to_np(mine))
    P1 = kmin.shape[2] - 1
    slopes = np.repeat(slopes_kv, G).astype(np.float32) if alibi else None
    ref = O.page_criticality(q[:, :, 0], kmin, kmax, dtype, num_pages=P1, alibi_slopes=slopes,
                             page_size=ps, seq_len=S, q_pos=S - 1)
    # fp32 summation order differs from the float64 oracle: 2^-20 of the
    # magnitudes summed, then one rounding to the dtype
    terms = np.abs(O.page_criticality(q[:, :, 0], kmin, kmax, "fp32", num_pages=P1))
    if alibi:
        terms = terms + np.abs(O.alibi_page_bonus(slopes, P1, ps, S, S - 1))[None]
    ulp = {"fp16": 2.0 ** -10, "bf16": 2.0 ** -7, "fp32": 2.0 ** -23}[dtype]
    assert (np.abs(to_np(got) - ref) <= 2.0 ** -20 * terms + ulp * np.abs(ref)).all()
