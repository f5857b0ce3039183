"""Accuracy of the GQA selection policies on the GPU against dense exact entmax
(the query heads of a group want different pages and differ in scale).

Top-k: the group's table holds the k pages of best rank over its query
heads; the HIP step's error equals the oracle's for that table and stays
within the reference test's bar (1 - coverage) * 2 (tests/test_topk.py:177).
Gaussian: the group's table is the union of its heads' selections; its error
is at most that of selecting per query head (the table of an MHA-expanded
cache) and within the reference bar 0.5 (tests/test_gaussian.py:168).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import entmaxkv_oracle as O
from tests.gpu_helpers import (dense_entmax_attention, gqa_structured_case, rel_error, to_dev,
                               to_np)

pytestmark = pytest.mark.gpu


def _case(**kw):
    print("CASE", " ".join(f"{k}={v}" for k, v in kw.items()), flush=True)


# (B, Hkv, G): "split" few heads (criticality + top-k, then the decode);
# "head" B * Hkv >= 128 (one fused launch)
SHAPES = {"split": (2, 2, 4), "head": (8, 16, 2)}


@pytest.mark.parametrize("path", ["split", "head"])
@pytest.mark.parametrize("coverage", [0.05, 0.25])
def test_gqa_topk_accuracy(path, coverage):
    from entmaxkv_amd import PagedKVCache, sparse_attention_decode_paged
    _case(test="gqa_topk_accuracy", path=path, coverage=coverage)
    dtype, ps, D, S = "fp16", 16, 128, 4097
    B, Hkv, G = SHAPES[path]
    H = Hkv * G
    rng = np.random.default_rng(60)
    q, K, V = gqa_structured_case(rng, B, Hkv, G, S, D, ps, dtype, 3, 2, 3.0)
    cache = PagedKVCache(page_size=ps)
    cache.initialize(to_dev(K[:, :, :S - 1], dtype), to_dev(V[:, :, :S - 1], dtype))
    P = (S + ps - 1) // ps
    budget = max(1, int((coverage * S + ps - 1) // ps)) * ps
    n_sel = min(budget // ps, P - 1)
    out = torch.zeros(B, H, 1, D, dtype=torch.float16, device="cuda")
    sparse_attention_decode_paged(
        to_dev(q[:, :, None], dtype), cache, to_dev(K[:, :, S - 1:], dtype),
        to_dev(V[:, :, S - 1:], dtype), out, budget,
        torch.full((B,), n_sel * ps + 1, dtype=torch.int32, device="cuda"),
        torch.full((B,), S, dtype=torch.int32, device="cuda"), alpha=1.5, niter=10)
    torch.cuda.synchronize()
    pidx = to_np(cache._page_indices_buf).astype(np.int64)
    sel = O.topk_gqa_pages(to_np(cache.last_page_scores), Hkv, n_sel)
    np.testing.assert_array_equal(pidx[:, :, :n_sel], sel)
    ref = dense_entmax_attention(q, K, V, 1.5, dtype)
    got = rel_error(to_np(out)[:, :, 0], ref)
    want = rel_error(O.paged_entmax_decode(q, K, V, pidx, np.full((B, Hkv), n_sel * ps + 1), ps,
                                           1.5, 10, dtype)[0], ref)
    print(f"rel_error {got:.4f} (oracle {want:.4f})", flush=True)
    assert abs(got - want) < 2e-3
    assert got < (1.0 - coverage) * 2.0


def test_gqa_gaussian_union_accuracy():
    from entmaxkv_amd import PagedKVCache, sparse_attention_decode_gaussian_aware_entmax
    _case(test="gqa_gaussian_accuracy")
    dtype, ps, D, S = "fp16", 16, 128, 4096
    B, Hkv, G = 2, 2, 4
    H = Hkv * G
    rng = np.random.default_rng(61)
    q, K, V = gqa_structured_case(rng, B, Hkv, G, S, D, ps, dtype, 3, 2, 6.0)
    cache = PagedKVCache(page_size=ps)
    cache.initialize(to_dev(K, dtype), to_dev(V, dtype))
    out = torch.zeros(B, H, 1, D, dtype=torch.float16, device="cuda")
    sparse_attention_decode_gaussian_aware_entmax(to_dev(q[:, :, None], dtype), cache, None, None,
                                                  out, alpha=1.5, tau_mode="exact")
    torch.cuda.synchronize()
    ref = dense_entmax_attention(q, K, V, 1.5, dtype)
    got = rel_error(to_np(out)[:, :, 0], ref)
    # per query head: the same step on an MHA-expanded cache
    kmean, kstd = O.page_stats(K, ps, dtype)[2:4]
    per_head = O.gaussian_decode_step(q, np.repeat(K, G, 1), np.repeat(V, G, 1),
                                      np.repeat(kmean, G, 1), np.repeat(kstd, G, 1), ps, 1.5,
                                      dtype, tau_mode="exact")
    want = rel_error(per_head["out"], ref)
    counts = to_np(cache.last_num_selected_per_head)
    print(f"rel_error {got:.4f} (per head {want:.4f}); pages {counts.mean():.1f} of "
          f"{S // ps} (per head {per_head['counts'].mean():.1f})", flush=True)
    assert got <= want + 2e-3
    assert got < 0.5
