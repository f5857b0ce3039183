"""Block-pool KV layout (PagedKVCache(block_pool=True)) on the GPU.

The reference keeps one contiguous cache per batch (kv_cache.py:23-38); the
block pool with its block table is this build's extension.  A decode step
reads the same K/V values in the same order whichever layout holds them, so
every output of the pool mode (decode output, page tables, page scores,
statistics, the gathered K/V) must equal the contiguous mode's bit for bit,
step after step with appends, while the table and the pool both grow.  The
contiguous mode is pinned against the oracle elsewhere; one case here also
checks the pool mode against the oracle directly.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import entmaxkv_oracle as O
from tests.gpu_helpers import TORCH_DT, assert_out_close, randn, to_dev, to_np
from tests.test_gpu_parity import _case, _gqa_gaussian_inputs

pytestmark = pytest.mark.gpu


def _pair(k, v, dtype, lens, S):
    """(contiguous cache, block-pool cache) holding the same prefill.  The
    pool starts a block short of what the appends need and the table at
    S + 1 rows, so both grow during the test."""
    from entmaxkv_amd import PagedKVCache
    B = k.shape[0]
    seq = torch.tensor(lens) if lens is not None else None
    ref = PagedKVCache(page_size=16)
    ref.initialize(to_dev(k, dtype), to_dev(v, dtype), seq_lens=seq)
    n = [(x + 15) // 16 for x in (lens if lens is not None else [S] * B)]
    pool = PagedKVCache(page_size=16, capacity=S + 1, block_pool=True, num_blocks=sum(n) + 1)
    pool.initialize(to_dev(k, dtype), to_dev(v, dtype), seq_lens=seq)
    return ref, pool


def _same(a, b, what):
    torch.cuda.synchronize()
    assert a.shape == b.shape, what
    assert torch.equal(a, b), f"{what}: block pool differs from the contiguous cache"


def _compare_caches(ref, pool):
    assert pool.seq_len == ref.seq_len
    for name in ("k_min", "k_max", "k_mean", "k_std", "k_cache", "v_cache"):
        a, b = getattr(ref, name), getattr(pool, name)
        if ref.is_ragged:
            # rows past a sequence's own length are unspecified in either layout
            lens = ref.seq_lens.tolist()
            for i, n in enumerate(lens):
                rows = n if name.endswith("cache") else (n + 15) // 16
                _same(a[i, :, :rows], b[i, :, :rows], name)
        else:
            _same(a, b, name)


def _interleaved(pool, B):
    """The table hands blocks out page-major, so sequences interleave."""
    t = pool.block_table[:, :2].cpu()
    return B == 1 or int(t[1, 0]) == 1


@pytest.mark.parametrize("path,G,dtype,ragged", [("head", 1, "fp16", False),
                                                 ("head", 4, "bf16", True),
                                                 ("split", 2, "fp32", False),
                                                 ("split", 1, "bf16", True)])
def test_block_pool_topk_steps(path, G, dtype, ragged):
    from entmaxkv_amd import sparse_attention_decode_paged
    _case(test="block_pool_topk", path=path, G=G, dtype=dtype, ragged=ragged)
    rng = np.random.default_rng(91 + G)
    B, Hkv = (8, 16) if path == "head" else (3, 2)
    S, D, budget = 16 * 40 - 1, 64, 192  # the first append completes a page
    H = Hkv * G
    k = randn(rng, (B, Hkv, S, D), dtype)
    v = randn(rng, (B, Hkv, S, D), dtype)
    q = randn(rng, (B, H, 1, D), dtype)
    lens = None
    if ragged:
        lens = [int(x) for x in rng.integers(20, S, B)]
        lens[0], lens[-1] = S, 31
    ref, pool = _pair(k, v, dtype, lens, S)
    assert _interleaved(pool, B)
    for step in range(4):
        kn = to_dev(randn(rng, (B, Hkv, 1, D), dtype), dtype)
        vn = to_dev(randn(rng, (B, Hkv, 1, D), dtype), dtype)
        outs = []
        for c in (ref, pool):
            out = torch.zeros(B, H, 1, D, dtype=TORCH_DT[dtype], device="cuda")
            sparse_attention_decode_paged(to_dev(q, dtype), c, kn, vn, out, budget, None, None,
                                          alpha=1.5 if step % 2 == 0 else 2.0, niter=10)
            outs.append(out)
        _same(outs[0], outs[1], f"out step {step}")
        if ragged:
            # sequence b fills slots 0 .. k_b (its last page at k_b); the rest is unspecified
            for i, n in enumerate(ref.seq_lens.tolist()):
                k_b = min(budget // 16, (n + 15) // 16 - 1)
                _same(ref._page_indices_buf[i, :, :k_b + 1], pool._page_indices_buf[i, :, :k_b + 1],
                      f"page table step {step}")
        else:
            _same(ref._page_indices_buf, pool._page_indices_buf, f"page table step {step}")
        if ragged:
            for i, n in enumerate(ref.seq_lens.tolist()):
                P_b = (n + 15) // 16
                _same(ref.last_page_scores[i, :, :P_b - 1], pool.last_page_scores[i, :, :P_b - 1],
                      f"scores step {step}")
        else:
            _same(ref.last_page_scores, pool.last_page_scores, f"scores step {step}")
        _compare_caches(ref, pool)
    assert pool.block_table.shape[1] > (S + 1 + 15) // 16  # the table grew
    if not ragged and path == "head" and G == 1:
        # the pool mode against the oracle on the last step's state
        ps, alpha, S_b = 16, 2.0, pool.seq_len
        P = (S_b + ps - 1) // ps
        n_sel = min(budget // ps, P - 1)
        kf, vf = to_np(pool.k_cache), to_np(pool.v_cache)
        st = O.page_stats(kf, ps, dtype)
        scores = to_np(pool.last_page_scores)
        sel = O.topk_gqa_pages(scores, Hkv, n_sel)
        pidx = np.concatenate([sel, np.full((B, Hkv, 1), P - 1)], axis=2)
        np.testing.assert_array_equal(to_np(pool._page_indices_buf).astype(np.int64), pidx)
        np.testing.assert_array_equal(to_np(pool.k_min), st[0])
        lps = S_b - (P - 1) * ps
        want, _ = O.paged_entmax_decode(q[:, :, 0], kf, vf, pidx,
                                        np.full((B, Hkv), n_sel * ps + lps), ps, alpha, 10, dtype)
        assert_out_close(to_np(outs[1])[:, :, 0], want, dtype)


def test_block_pool_dense_step():
    """budget < page_size: no page selection, the last page alone (k = 0)."""
    from entmaxkv_amd import sparse_attention_decode_paged
    _case(test="block_pool_dense")
    dtype = "bf16"
    rng = np.random.default_rng(95)
    B, Hkv, G, S, D = 4, 4, 2, 16 * 8 + 3, 128
    k = randn(rng, (B, Hkv, S, D), dtype)
    v = randn(rng, (B, Hkv, S, D), dtype)
    q = randn(rng, (B, Hkv * G, 1, D), dtype)
    ref, pool = _pair(k, v, dtype, None, S)
    kn = to_dev(randn(rng, (B, Hkv, 1, D), dtype), dtype)
    vn = to_dev(randn(rng, (B, Hkv, 1, D), dtype), dtype)
    outs = []
    for c in (ref, pool):
        out = torch.zeros(B, Hkv * G, 1, D, dtype=TORCH_DT[dtype], device="cuda")
        sparse_attention_decode_paged(to_dev(q, dtype), c, kn, vn, out, 8, None, None, alpha=1.5)
        outs.append(out)
    _same(outs[0], outs[1], "out")
    _compare_caches(ref, pool)


@pytest.mark.parametrize("path,G,tau_mode,ragged", [("head", 4, "corrected", False),
                                                    ("head", 1, "exact", True),
                                                    ("split", 2, "fixed", True)])
def test_block_pool_gaussian_steps(path, G, tau_mode, ragged):
    from entmaxkv_amd import sparse_attention_decode_gaussian_aware_entmax
    _case(test="block_pool_gaussian", path=path, G=G, tau_mode=tau_mode, ragged=ragged)
    dtype, alpha = "bf16", 1.5
    rng = np.random.default_rng(97 + G)
    B, Hkv = (8, 16) if path == "head" else (3, 2)
    S, D = 16 * 60 - 2, 128
    H = Hkv * G
    q, k, v = _gqa_gaussian_inputs(rng, dtype, B, Hkv, G, S, D, 0.03)
    lens = None
    if ragged:
        lens = [int(x) for x in rng.integers(40, S, B)]
        lens[0], lens[-1] = S, 33
    ref, pool = _pair(k, v, dtype, lens, S)
    for step in range(3):
        kn = to_dev(randn(rng, (B, Hkv, 1, D), dtype), dtype)
        vn = to_dev(randn(rng, (B, Hkv, 1, D), dtype), dtype)
        outs, stats = [], []
        for c in (ref, pool):
            out = torch.zeros(B, H, 1, D, dtype=TORCH_DT[dtype], device="cuda")
            st = sparse_attention_decode_gaussian_aware_entmax(
                to_dev(q, dtype), c, kn, vn, out, alpha=alpha, tau_mode=tau_mode,
                append_cache=True)
            outs.append(out)
            stats.append(c.last_num_selected_per_head.clone())
        _same(outs[0], outs[1], f"out step {step}")
        _same(stats[0], stats[1], f"selected pages step {step}")
        _compare_caches(ref, pool)
