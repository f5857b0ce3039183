"""Decode steps captured in a hipGraph (torch.cuda.CUDAGraph) and replayed.

Serving loops capture the decode step once and replay it; bench.py times
replays too.  Every replay must give the eager step's outputs bit for bit,
with eager work and host synchronisations between the replays (the step
launches no memset and allocates nothing once its buffers exist).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from tests.gpu_helpers import TORCH_DT, randn, to_dev
from tests.test_gpu_parity import _case, _gqa_gaussian_inputs

pytestmark = pytest.mark.gpu


def _replays_match(step, outputs, n=3):
    """Eager reference, one capture, n replays separated by unrelated eager
    work; every replay's outputs equal the eager ones."""
    step()
    torch.cuda.synchronize()
    want = [o.clone() for o in outputs]
    for o in outputs:
        o.fill_(float("nan")) if o.is_floating_point() else o.fill_(-7)
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        step()  # warm the side stream (no allocation happens in the capture)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    with torch.cuda.graph(g):
        step()
    for r in range(n):
        for o in outputs:
            o.fill_(float("nan")) if o.is_floating_point() else o.fill_(-7)
        junk = torch.randn(1 << 20, device="cuda").sum()  # eager work between replays
        g.replay()
        torch.cuda.synchronize()
        assert torch.isfinite(junk)
        for o, w in zip(outputs, want):
            assert torch.equal(o, w), f"replay {r} differs from the eager step"


@pytest.mark.parametrize("B,Hkv,G,dtype", [(8, 32, 1, "fp16"), (4, 32, 1, "fp16"),
                                           (16, 8, 4, "bf16"), (2, 2, 2, "fp16")])
def test_topk_step_graph_replay(B, Hkv, G, dtype):
    """Fused scan (B*Hkv = 256), prescored (128), GQA prescored, split path."""
    from entmaxkv_amd import PagedKVCache, sparse_attention_decode_paged
    _case(test="graph_topk", B=B, Hkv=Hkv, G=G, dtype=dtype)
    rng = np.random.default_rng(601)
    S, D, budget = 16 * 80 + 1, 128, 256
    k = randn(rng, (B, Hkv, S, D), dtype)
    v = randn(rng, (B, Hkv, S, D), dtype)
    q = to_dev(randn(rng, (B, Hkv * G, 1, D), dtype), dtype)
    cache = PagedKVCache(page_size=16)
    cache.initialize(to_dev(k, dtype), to_dev(v, dtype))
    out = torch.zeros(B, Hkv * G, 1, D, dtype=TORCH_DT[dtype], device="cuda")

    def step():
        sparse_attention_decode_paged(q, cache, None, None, out, budget, None, None, alpha=1.5,
                                      niter=2, append_cache=False)
    step()  # allocates the cache's buffers before any capture
    torch.cuda.synchronize()
    _replays_match(step, [out, cache._page_indices_buf])


@pytest.mark.parametrize("B,Hkv,G,tau_mode", [(8, 32, 1, "corrected"), (4, 32, 1, "exact"),
                                               (4, 8, 4, "corrected")])
def test_gaussian_step_graph_replay(B, Hkv, G, tau_mode):
    from entmaxkv_amd import PagedKVCache, sparse_attention_decode_gaussian_aware_entmax
    _case(test="graph_gaussian", B=B, Hkv=Hkv, G=G, tau_mode=tau_mode)
    dtype = "fp16" if G == 1 else "bf16"
    rng = np.random.default_rng(602)
    S, D = 16 * 70 - 3, 128
    qn, k, v = _gqa_gaussian_inputs(rng, dtype, B, Hkv, G, S, D, 0.03)
    q = to_dev(qn, dtype)
    cache = PagedKVCache(page_size=16)
    cache.initialize(to_dev(k, dtype), to_dev(v, dtype))
    out = torch.zeros(B, Hkv * G, 1, D, dtype=TORCH_DT[dtype], device="cuda")

    def step():
        sparse_attention_decode_gaussian_aware_entmax(q, cache, None, None, out, alpha=1.5,
                                                      tau_mode=tau_mode, append_cache=False)
    step()
    torch.cuda.synchronize()
    _replays_match(step, [out, cache.last_num_selected_per_head])
