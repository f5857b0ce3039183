"""The top-k step with append_cache=True writes the new row inside its own
launch (ekv_append_topk_paged_entmax_decode) for a uniform batch.  It must
leave the cache and give the outputs of the two-call sequence the reference
runs (kv_cache.py:72-116, then attention_topk.py:52-98): here the explicit
``append`` followed by the step with append_cache=False, bit for bit, over
several steps that cross page boundaries, on the fused, prescored and split
launch paths, with and without the block pool.  The two-call sequence itself
is pinned against the oracle by the parity tests.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from tests.gpu_helpers import TORCH_DT, randn, to_dev
from tests.test_gpu_parity import _case

pytestmark = pytest.mark.gpu


def _same(a, b, what):
    torch.cuda.synchronize()
    assert a.shape == b.shape, what
    assert torch.equal(a, b), f"{what}: fused append differs from append + step"


@pytest.mark.parametrize("B,Hkv,G,dtype,pool,budget,alibi", [
    (8, 32, 1, "fp16", False, 256, False),   # fused scan (B * Hkv = 256)
    (8, 32, 1, "fp16", False, 256, True),    # ALiBi
    (4, 32, 1, "fp16", False, 256, False),   # prescored (128)
    (16, 8, 4, "bf16", False, 512, False),   # GQA, prescored
    (2, 2, 2, "fp32", False, 128, False),    # split launches (the append runs first)
    (2, 2, 2, "fp32", False, 128, True),     # split launches, ALiBi
    (8, 16, 1, "bf16", True, 256, False),    # block pool
    (4, 4, 2, "fp16", False, 8, False),      # budget below a page: no selection
])
def test_fused_append_matches_append_then_step(B, Hkv, G, dtype, pool, budget, alibi):
    from entmaxkv_amd import PagedKVCache, sparse_attention_decode_paged
    _case(test="fused_append", B=B, Hkv=Hkv, G=G, dtype=dtype, pool=pool, budget=budget,
          alibi=alibi)
    rng = np.random.default_rng(700 + B + G)
    S, D = 16 * 24 - 2, 128  # the second append completes a page, the third opens one
    H = Hkv * G
    k = randn(rng, (B, Hkv, S, D), dtype)
    v = randn(rng, (B, Hkv, S, D), dtype)
    q = to_dev(randn(rng, (B, H, 1, D), dtype), dtype)
    caches = []
    for _ in range(2):
        c = PagedKVCache(page_size=16, capacity=S + 2, block_pool=pool,
                         num_blocks=B * 25 if pool else None)
        c.initialize(to_dev(k, dtype), to_dev(v, dtype))
        caches.append(c)
    fused, ref = caches
    slopes = (torch.tensor([2.0 ** (-8.0 * (h + 1) / H) for h in range(H)], device="cuda")
              if alibi else None)
    for step in range(5):
        kn = to_dev(randn(rng, (B, Hkv, 1, D), dtype), dtype)
        vn = to_dev(randn(rng, (B, Hkv, 1, D), dtype), dtype)
        outs = [torch.zeros(B, H, 1, D, dtype=TORCH_DT[dtype], device="cuda") for _ in range(2)]
        sparse_attention_decode_paged(q, fused, kn, vn, outs[0], budget, None, None,
                                      alibi_slopes=slopes, alpha=1.5, niter=2,
                                      append_cache=True)
        ref.append(kn, vn)
        sparse_attention_decode_paged(q, ref, None, None, outs[1], budget, None, None,
                                      alibi_slopes=slopes, alpha=1.5, niter=2,
                                      append_cache=False)
        assert fused.seq_len == ref.seq_len == S + step + 1
        _same(outs[0], outs[1], f"out step {step}")
        _same(fused._page_indices_buf, ref._page_indices_buf, f"page table step {step}")
        for name in ("k_min", "k_max", "k_mean", "k_std", "k_cache", "v_cache"):
            _same(getattr(fused, name), getattr(ref, name), f"{name} step {step}")
