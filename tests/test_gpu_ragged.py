"""Ragged batches (per-sequence lengths) on the GPU against the oracle.

The reference cache holds one length (kv_cache.py:23-38), so a ragged batch
is this build's extension (benchmark config 5).  It is pinned by per-sequence
decomposition: every sequence must give what the oracle gives for that
sequence alone, except for the batch-wide automatic margins of the Gaussian
selection, which are formed from every head of the batch as in the uniform
case (gaussian_utils.py:163-169).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import entmaxkv_oracle as O
from tests.gpu_helpers import TORCH_DT, assert_out_close, randn, to_dev, to_np, ulp_diff_16
from tests.test_gpu_parity import _case, _check_gaussian_step, _gqa_gaussian_inputs

pytestmark = pytest.mark.gpu


def _ragged_cache(k, v, lens, dtype):
    from entmaxkv_amd import PagedKVCache
    cache = PagedKVCache(page_size=16)
    cache.initialize(to_dev(k, dtype), to_dev(v, dtype), seq_lens=torch.tensor(lens))
    return cache


def _with_appended(k, kn, lens):
    """k [B, Hkv, S, D] with each sequence's new row written at its own length."""
    B, Hkv, S, D = k.shape
    out = np.concatenate([k, np.zeros((B, Hkv, 1, D))], axis=2)
    for b in range(B):
        out[b, :, lens[b]] = kn[b, :, 0]
    return out


@pytest.mark.parametrize("dtype", ["fp16", "fp32"])
def test_ragged_stats_and_append(dtype):
    _case(test="ragged_stats", dtype=dtype)
    rng = np.random.default_rng(71)
    B, Hkv, S, D, ps = 3, 4, 100, 64, 16
    lens = [37, 100, 64]
    k = randn(rng, (B, Hkv, S, D), dtype)
    v = randn(rng, (B, Hkv, S, D), dtype)
    cache = _ragged_cache(k, v, lens, dtype)
    for step in range(3):
        if step:
            kn = randn(rng, (B, Hkv, 1, D), dtype)
            vn = randn(rng, (B, Hkv, 1, D), dtype)
            cache.append(to_dev(kn, dtype), to_dev(vn, dtype))
            k = _with_appended(k, kn, lens)
            v = _with_appended(v, vn, lens)
            lens = [n + 1 for n in lens]
        torch.cuda.synchronize()
        assert to_np(cache.seq_lens).astype(int).tolist() == lens
        assert cache.seq_len == max(lens)
        got = [to_np(t) for t in (cache.k_min, cache.k_max, cache.k_mean, cache.k_std)]
        for b in range(B):
            P = (lens[b] + ps - 1) // ps
            ref = O.page_stats(k[b:b + 1, :, :lens[b]], ps, dtype)
            for j in range(4):
                g = got[j][b:b + 1, :, :P]
                if j < 2:
                    np.testing.assert_array_equal(g, ref[j])
                elif dtype == "fp32":
                    # fp32 accumulation of <= 16 rows of O(1) values vs the float64 oracle
                    np.testing.assert_allclose(g, ref[j], atol=2e-6, rtol=1e-6)
                else:
                    assert ulp_diff_16(g, ref[j], dtype).max() <= 1.0
            np.testing.assert_array_equal(to_np(cache.k_cache)[b, :, :lens[b]], k[b, :, :lens[b]])


# "head": one fused launch (B * Hkv = 128); "split": separate launches
@pytest.mark.parametrize("path,G,dtype", [("head", 1, "fp16"), ("head", 4, "bf16"),
                                          ("split", 2, "fp32")])
def test_ragged_topk_step(path, G, dtype):
    from entmaxkv_amd import sparse_attention_decode_paged
    _case(test="ragged_topk", path=path, G=G, dtype=dtype)
    rng = np.random.default_rng(72 + G)
    B, Hkv = (8, 16) if path == "head" else (3, 2)
    S, D, ps, budget = 1600, 64, 16, 256
    H = Hkv * G
    lens = [int(x) for x in rng.integers(20, S, B)]
    lens[0] = S
    lens[-1] = 17  # two pages: one scored page, k_b = 1
    k = randn(rng, (B, Hkv, S, D), dtype)
    v = randn(rng, (B, Hkv, S, D), dtype)
    q = randn(rng, (B, H, 1, D), dtype)
    kn = randn(rng, (B, Hkv, 1, D), dtype)
    vn = randn(rng, (B, Hkv, 1, D), dtype)
    cache = _ragged_cache(k, v, lens, dtype)
    out = torch.zeros(B, H, 1, D, dtype=TORCH_DT[dtype], device="cuda")
    sparse_attention_decode_paged(to_dev(q, dtype), cache, to_dev(kn, dtype), to_dev(vn, dtype),
                                  out, budget, None, None, alpha=1.5, niter=10)
    torch.cuda.synchronize()
    kf, vf = _with_appended(k, kn, lens), _with_appended(v, vn, lens)
    lens = [n + 1 for n in lens]
    scores_all = to_np(cache.last_page_scores)
    table = to_np(cache._page_indices_buf).astype(np.int64)
    got = to_np(out)[:, :, 0]
    for b in range(B):
        S_b = lens[b]
        P = (S_b + ps - 1) // ps
        n_sel = min(budget // ps, P - 1)
        st = O.page_stats(kf[b:b + 1, :, :S_b], ps, dtype)
        scores = scores_all[b:b + 1, :, :P - 1]
        ref_scores = O.page_criticality(q[b:b + 1, :, 0], st[0], st[1], dtype, num_pages=P - 1)
        terms = np.abs(O.page_criticality(q[b:b + 1, :, 0], st[0], st[1], "fp32", num_pages=P - 1))
        ulp = {"fp16": 2.0 ** -10, "bf16": 2.0 ** -7, "fp32": 2.0 ** -23}[dtype]
        assert (np.abs(scores - ref_scores) <= 2.0 ** -20 * terms + ulp * np.abs(ref_scores)).all()
        sel = O.topk_gqa_pages(scores, Hkv, n_sel)
        pidx = np.concatenate([sel, np.full((1, Hkv, 1), P - 1)], axis=2)
        np.testing.assert_array_equal(table[b:b + 1, :, :n_sel + 1], pidx)
        lps = S_b - (P - 1) * ps
        ref, _ = O.paged_entmax_decode(q[b:b + 1, :, 0], kf[b:b + 1, :, :S_b], vf[b:b + 1, :, :S_b],
                                       pidx, np.full((1, Hkv), n_sel * ps + lps), ps, 1.5, 10,
                                       dtype)
        assert_out_close(got[b:b + 1], ref, dtype)


# config 5 in miniature: GQA, Gaussian alpha 1.5, append_cache=True, several
# consecutive steps; "head" = one fused launch per step, "split" = few heads.
# D = 128 with G = 4 in bf16 is config 5's own head shape.
@pytest.mark.parametrize("path,G,tau_mode,D", [("head", 4, "corrected", 64), ("head", 1, "exact", 64),
                                               ("split", 2, "corrected", 64),
                                               ("head", 4, "corrected", 128),
                                               ("split", 4, "corrected", 128)])
def test_ragged_gaussian_steps(path, G, tau_mode, D):
    from entmaxkv_amd import sparse_attention_decode_gaussian_aware_entmax
    _case(test="ragged_gaussian", path=path, G=G, tau_mode=tau_mode, D=D)
    dtype, alpha = "bf16", 1.5
    rng = np.random.default_rng(81 + G)
    B, Hkv = (8, 16) if path == "head" else (3, 2)
    S = 16 * 90
    H = Hkv * G
    q, k, v = _gqa_gaussian_inputs(rng, dtype, B, Hkv, G, S, D, 0.03)
    lens = [int(x) for x in rng.integers(40, S - 3, B)]
    lens[0] = S - 3
    lens[-1] = 33
    cache = _ragged_cache(k, v, lens, dtype)
    for step in range(3):
        kn = randn(rng, (B, Hkv, 1, D), dtype)
        vn = randn(rng, (B, Hkv, 1, D), dtype)
        out = torch.zeros(B, H, 1, D, dtype=TORCH_DT[dtype], device="cuda")
        sparse_attention_decode_gaussian_aware_entmax(
            to_dev(q, dtype), cache, to_dev(kn, dtype), to_dev(vn, dtype), out, alpha=alpha,
            tau_mode=tau_mode, append_cache=True)
        torch.cuda.synchronize()
        k, v = _with_appended(k, kn, lens), _with_appended(v, vn, lens)
        lens = [n + 1 for n in lens]
        _check_gaussian_step(cache, q, k, v, out, dtype, G, tau_mode, alpha, lens)
