"""The bound and moment scans alternate their page order from one launch to the
next (consecutive decode steps then start with the pages the last one read
most recently, which the GPU's memory-side cache still holds).  The order must
not change any result: two consecutive launches on the same inputs, which run
in opposite orders, give the same bits.  Shapes cover the fused scan (B * Hkv
= 256), the paired launch (128, G = 1), the prescored scan launch (128,
G = 4), and moment scans whose last round is partial.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from tests.gpu_helpers import TORCH_DT, randn, to_dev
from tests.test_gpu_parity import _case

pytestmark = pytest.mark.gpu


def _equal(a, b, what):
    torch.cuda.synchronize()
    assert a.shape == b.shape, what
    assert torch.equal(a, b), f"{what}: differs between two consecutive launches"


@pytest.mark.parametrize("B,Hkv,G,P,dtype", [(8, 16, 4, 61, "bf16"), (8, 16, 4, 60, "bf16"),
                                             (3, 2, 4, 61, "bf16"), (8, 32, 1, 2048, "fp16"),
                                             (4, 8, 2, 333, "fp32")])
def test_moments_same_bits_in_both_orders(B, Hkv, G, P, dtype):
    from entmaxkv_amd.kernels import GaussianBuffers, compute_page_gaussian_moments
    _case(test="moments_order", B=B, Hkv=Hkv, G=G, P=P, dtype=dtype)
    rng = np.random.default_rng(800 + P)
    H, D = Hkv * G, 128 if dtype != "fp32" else 64
    q = to_dev(randn(rng, (B, H, 1, D), dtype), dtype)
    km = to_dev(randn(rng, (B, Hkv, P + 3, D), dtype), dtype)
    ks = to_dev(np.abs(randn(rng, (B, Hkv, P + 3, D), dtype)), dtype)
    dev = torch.device("cuda:0")
    bufs = []
    for _ in range(3):
        buf = GaussianBuffers(B, H, Hkv, D, P, TORCH_DT[dtype], dev)
        compute_page_gaussian_moments(q, km, ks, P, buf, page_size=16, seq_len=P * 16)
        bufs.append(buf)
    for other in bufs[1:]:
        _equal(bufs[0].mu_p, other.mu_p, "mu_p")
        _equal(bufs[0].sigma_p, other.sigma_p, "sigma_p")
        _equal(bufs[0].ws, other.ws, "partial sums")


@pytest.mark.parametrize("B,Hkv,G,dtype", [(8, 32, 1, "fp16"), (4, 32, 1, "fp16"),
                                           (16, 8, 4, "bf16"), (8, 16, 2, "fp16")])
def test_topk_step_same_bits_in_both_orders(B, Hkv, G, dtype):
    from entmaxkv_amd import PagedKVCache, sparse_attention_decode_paged
    _case(test="topk_order", B=B, Hkv=Hkv, G=G, dtype=dtype)
    rng = np.random.default_rng(810 + B)
    S, D, budget = 16 * 150 + 5, 128, 512
    H = Hkv * G
    k = randn(rng, (B, Hkv, S, D), dtype)
    v = randn(rng, (B, Hkv, S, D), dtype)
    q = to_dev(randn(rng, (B, H, 1, D), dtype), dtype)
    cache = PagedKVCache(page_size=16)
    cache.initialize(to_dev(k, dtype), to_dev(v, dtype))
    got = []
    for _ in range(3):
        out = torch.zeros(B, H, 1, D, dtype=TORCH_DT[dtype], device="cuda")
        sparse_attention_decode_paged(q, cache, None, None, out, budget, None, None, alpha=1.5,
                                      niter=2, append_cache=False)
        torch.cuda.synchronize()
        got.append((out, cache._page_indices_buf.clone()))
    for out, table in got[1:]:
        _equal(got[0][0], out, "out")
        _equal(got[0][1], table, "page table")


@pytest.mark.parametrize("B,Hkv,G,fill", [(4, 32, 1, "random"), (4, 32, 1, "ones"),
                                          (8, 16, 2, "random")])
def test_paired_topk_any_workspace(B, Hkv, G, fill):
    """B * Hkv = 128 with groups of at most 2 runs the paired launch (two
    workgroups per (b, kv head) scanning half of its pages each); its arrival
    words live in the decode workspace, which a caller need not initialise.
    Random bytes, or every byte 0xff, in the workspace between steps leave
    the results unchanged."""
    from entmaxkv_amd import PagedKVCache, sparse_attention_decode_paged
    _case(test="paired_workspace", B=B, Hkv=Hkv, G=G, fill=fill)
    dtype = "fp16"
    rng = np.random.default_rng(820)
    S, D, budget = 16 * 200 + 9, 128, 1024
    k = randn(rng, (B, Hkv, S, D), dtype)
    v = randn(rng, (B, Hkv, S, D), dtype)
    q = to_dev(randn(rng, (B, Hkv * G, 1, D), dtype), dtype)
    cache = PagedKVCache(page_size=16)
    cache.initialize(to_dev(k, dtype), to_dev(v, dtype))
    got = []
    for step in range(3):
        for ws in cache._paged_decode_workspaces.values():
            if fill == "random":
                ws.buf.copy_(torch.randint(0, 256, ws.buf.shape, dtype=torch.uint8))
            else:
                ws.buf.fill_(255)
        out = torch.zeros(B, Hkv * G, 1, D, dtype=TORCH_DT[dtype], device="cuda")
        sparse_attention_decode_paged(q, cache, None, None, out, budget, None, None, alpha=1.5,
                                      niter=2, append_cache=False)
        torch.cuda.synchronize()
        got.append((out, cache._page_indices_buf.clone()))
    assert torch.isfinite(got[0][0].float()).all()
    for out, table in got[1:]:
        _equal(got[0][0], out, "out")
        _equal(got[0][1], table, "page table")
