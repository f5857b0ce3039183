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


@pytest.mark.parametrize("shape", [(2, 2, 4, 400, 100, "bf16"), (8, 16, 1, 300, 64, "fp16")])
def test_noalloc_step_graph_replay(shape):
    """ekv_topk_paged_entmax_decode_noalloc, the entry point for code under
    graph capture (its workspace is the library's static scratch)."""
    from entmaxkv_amd import _lib
    from entmaxkv_amd.kernels import choose_splits, qscale_for
    from tests.test_zz_no_alloc import _case as noalloc_case
    B, Hkv, G, pages, k, dtype = shape
    _case(test="graph_noalloc", B=B, Hkv=Hkv, G=G, pages=pages, k=k, dtype=dtype)
    c = noalloc_case(B, Hkv, G, pages, k, dtype, 11)
    dev = c["q"].device
    H, D, ps, P = c["H"], c["D"], c["ps"], c["P"]
    dt = TORCH_DT[dtype]
    n_slots = k + 1
    max_tokens = n_slots * ps
    scores = torch.zeros((B, H, P - 1), dtype=dt, device=dev)
    pidx = torch.zeros((B, Hkv, n_slots), dtype=torch.int32, device=dev)
    seqlens = torch.full((B, Hkv), k * ps + c["lps"], dtype=torch.int32, device=dev)
    tau = torch.zeros((B, H), dtype=torch.float32, device=dev)
    out = torch.zeros((B, H, D), dtype=dt, device=dev)
    q3 = c["q"][:, :, 0]
    cache = c["cache"]
    kmin, kmax, kc, vc = cache.k_min, cache.k_max, cache._k, cache._v
    args = [q3.data_ptr(), q3.stride(0), q3.stride(1), kmin.data_ptr(), kmax.data_ptr(),
            kmin.stride(0), kmin.stride(1), kmin.stride(2), scores.data_ptr(), P - 1, c["S"],
            c["S"] - 1, k, P - 1, kc.data_ptr(), vc.data_ptr(), kc.stride(0), kc.stride(1),
            kc.stride(2), kc.shape[2], None, 0, 0, pidx.data_ptr(), pidx.stride(0),
            pidx.stride(1), seqlens.data_ptr(), seqlens.stride(0), seqlens.stride(1), None,
            None, None, tau.data_ptr(), 2, out.data_ptr(), out.stride(0), out.stride(1), 1.5,
            qscale_for(1.5, D, dt), ps, B, H, Hkv, D, choose_splits(max_tokens), max_tokens,
            {"fp32": 0, "fp16": 1, "bf16": 2}[dtype]]

    def step():
        _lib.call("ekv_topk_paged_entmax_decode_noalloc", *args,
                  torch.cuda.current_stream(dev).cuda_stream)
    _replays_match(step, [out, pidx, tau, scores])
