"""HIP path vs the CPU oracle on seeded inputs (needs an MI355X).

Every test prints the case it runs before touching the GPU so a failing run
names its case.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import entmaxkv_oracle as O
from tests.gpu_helpers import (ATOL, TORCH_DT, assert_out_close, randn, to_dev, to_np,
                               ulp_diff_16)

pytestmark = pytest.mark.gpu

DTYPES = ["fp16", "bf16", "fp32"]


def _case(**kw):
    print("CASE", " ".join(f"{k}={v}" for k, v in kw.items()), flush=True)


def _K():
    from entmaxkv_amd import kernels as K
    return K


# ---------------------------------------------------------------------------
# a1 / a2 page statistics
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("S", [1, 17, 1000])
def test_page_stats_initialize(dtype, S):
    from entmaxkv_amd import PagedKVCache
    _case(test="page_stats", dtype=dtype, S=S)
    rng = np.random.default_rng(S)
    B, H, D = 2, 3, 128
    k = randn(rng, (B, H, S, D), dtype)
    v = randn(rng, (B, H, S, D), dtype)
    cache = PagedKVCache(page_size=16)
    cache.initialize(to_dev(k, dtype), to_dev(v, dtype))
    torch.cuda.synchronize()
    ref = O.page_stats(k, 16, dtype)
    got = [cache.k_min, cache.k_max, cache.k_mean, cache.k_std]
    for name, g, r in zip(["min", "max", "mean", "std"], got, ref):
        g = to_np(g)
        assert g.shape == r.shape
        if name in ("min", "max"):
            np.testing.assert_array_equal(g, r)
        elif dtype == "fp32":
            # fp32 accumulation of <= 16 rows of O(1) values vs the float64 oracle
            np.testing.assert_allclose(g, r, atol=2e-6, rtol=1e-6, err_msg=name)
        else:
            assert ulp_diff_16(g, r, dtype).max() <= 1.0, name
    np.testing.assert_array_equal(to_np(cache.k_cache), k)
    np.testing.assert_array_equal(to_np(cache.v_cache), v)


@pytest.mark.parametrize("dtype", ["fp16", "bf16"])
def test_append_in_place_matches_rebuild(dtype):
    from entmaxkv_amd import PagedKVCache
    _case(test="append", dtype=dtype)
    rng = np.random.default_rng(3)
    B, H, D, S0, steps = 2, 4, 64, 30, 40
    k = randn(rng, (B, H, S0 + steps, D), dtype)
    v = randn(rng, (B, H, S0 + steps, D), dtype)
    cache = PagedKVCache(page_size=16, capacity=S0 + 8)  # forces a capacity growth
    kd, vd = to_dev(k, dtype), to_dev(v, dtype)
    cache.initialize(kd[:, :, :S0], vd[:, :, :S0])
    for t in range(S0, S0 + steps):
        cache.append(kd[:, :, t:t + 1], vd[:, :, t:t + 1])
    torch.cuda.synchronize()
    assert cache.k_cache.shape[2] == S0 + steps
    np.testing.assert_array_equal(to_np(cache.k_cache), k)
    np.testing.assert_array_equal(to_np(cache.v_cache), v)
    ref = O.page_stats(k, 16, dtype)
    for g, r in zip([cache.k_min, cache.k_max, cache.k_mean, cache.k_std], ref):
        assert ulp_diff_16(to_np(g), r, dtype).max() <= 1.0


# ---------------------------------------------------------------------------
# a3 / a4 criticality + top-k
# ---------------------------------------------------------------------------

def _build_cache(rng, B, Hkv, S, D, dtype, k_scale=1.0):
    from entmaxkv_amd import PagedKVCache
    k = randn(rng, (B, Hkv, S, D), dtype, k_scale)
    v = randn(rng, (B, Hkv, S, D), dtype)
    cache = PagedKVCache(page_size=16)
    cache.initialize(to_dev(k, dtype), to_dev(v, dtype))
    return cache, k, v


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("G", [1, 4])
@pytest.mark.parametrize("alibi", [False, True])
@pytest.mark.parametrize("path", ["split", "head"])
def test_criticality_and_topk(dtype, G, alibi, path):
    _case(test="criticality_topk", dtype=dtype, G=G, alibi=alibi, path=path)
    rng = np.random.default_rng(10 + G)
    B, Hkv = DECODE_SHAPES[path]
    S, D = 16 * 300 + 5, 128
    H = Hkv * G
    cache, k, v = _build_cache(rng, B, Hkv, S, D, dtype)
    q = randn(rng, (B, H, 1, D), dtype)
    qd = to_dev(q, dtype)
    slopes = None
    if alibi:
        slopes = np.exp2(-8.0 * np.arange(1, H + 1) / H).astype(np.float32)
    kk = 64
    pidx = cache.select_topk(qd, kk, alibi_slopes=None if slopes is None else torch.tensor(slopes, device="cuda"))
    torch.cuda.synchronize()
    P = cache.num_pages
    kmin, kmax = O.page_stats(k, 16, dtype)[:2]
    ref_scores = O.page_criticality(q[:, :, 0], kmin, kmax, dtype, num_pages=P - 1,
                                    alibi_slopes=slopes, page_size=16, seq_len=S, q_pos=S - 1)
    got_scores = to_np(cache.last_page_scores)
    # fp32 accumulation (order differs from the float64 oracle) is exact to
    # ~2^-20 of the magnitudes summed; the ALiBi bonus can cancel most of the
    # score, so the bound is taken on the terms, then one rounding to the dtype.
    plain = O.page_criticality(q[:, :, 0], kmin, kmax, "fp32", num_pages=P - 1)
    terms = np.abs(plain)
    if slopes is not None:
        terms = terms + np.abs(O.alibi_page_bonus(slopes, P - 1, 16, S, S - 1))[None]
    ulp = {"fp16": 2.0 ** -10, "bf16": 2.0 ** -7, "fp32": 2.0 ** -23}[dtype]
    tol = 2.0 ** -20 * terms + ulp * np.abs(ref_scores)
    assert (np.abs(got_scores - ref_scores) <= tol).all()
    # the page table is bit-exact given the scores the kernel produced
    ref_sel = O.topk_gqa_pages(got_scores, Hkv, kk)
    got = to_np(pidx).astype(np.int64)
    np.testing.assert_array_equal(got[:, :, :kk], ref_sel)
    assert (got[:, :, kk] == P - 1).all()


@pytest.mark.parametrize("dtype", DTYPES)
def test_topk_ties_and_edges(dtype):
    K = _K()
    _case(test="topk_ties", dtype=dtype)
    rng = np.random.default_rng(4)
    B, H, P = 2, 2, 1000
    s = O.round_to(np.round(rng.standard_normal((B, H, P)) * 4) / 4, dtype)  # many ties
    s[0, 0, 10] = np.nan
    sd = to_dev(s, dtype)
    for k in (0, 1, 37, 500, 999, 1000):
        out = K.topk_pages(sd, k, H, last_page=P)
        torch.cuda.synchronize()
        got = to_np(out).astype(np.int64)
        ref = O.topk_pages(s, k)
        np.testing.assert_array_equal(got[:, :, :k], ref, err_msg=f"k={k}")
        assert (got[:, :, k] == P).all()


@pytest.mark.parametrize("dtype", ["fp16", "bf16"])
@pytest.mark.parametrize("G", [2, 4, 8])
def test_topk_gqa_ties(dtype, G):
    """GQA page tables (best rank over the group) on tie-heavy scores: every
    head's top-k breaks ties toward the lower page, and so does the final
    selection over levels (compared with the oracle's policy)."""
    K = _K()
    _case(test="topk_gqa_ties", dtype=dtype, G=G)
    rng = np.random.default_rng(40 + G)
    B, Hkv, P = 2, 2, 1500
    H = Hkv * G
    s = O.round_to(np.round(rng.standard_normal((B, H, P)) * 3) / 4, dtype)
    sd = to_dev(s, dtype)
    for k in (1, 7, 64, 100, 128, 300, 1499):
        out = K.topk_pages(sd, k, Hkv, last_page=P)
        torch.cuda.synchronize()
        got = to_np(out).astype(np.int64)
        ref = O.topk_gqa_pages(s, Hkv, k)
        np.testing.assert_array_equal(got[:, :, :k], ref, err_msg=f"k={k}")
        assert (got[:, :, k] == P).all()


# ---------------------------------------------------------------------------
# a6 / a13 paged decode
# ---------------------------------------------------------------------------

def _decode_case(rng, dtype, B, Hkv, G, S, D, n_sel, k_scale=1.0):
    H = Hkv * G
    K_ = randn(rng, (B, Hkv, S, D), dtype, k_scale)
    V_ = randn(rng, (B, Hkv, S, D), dtype)
    q = randn(rng, (B, H, 1, D), dtype)
    P = (S + 15) // 16
    pidx = np.stack([np.stack([np.concatenate([np.sort(rng.choice(P - 1, n_sel, replace=False)), [P - 1]])
                               for _ in range(Hkv)]) for _ in range(B)])
    lps = S - (P - 1) * 16
    seqlens = np.full((B, Hkv), n_sel * 16 + lps)
    return K_, V_, q, pidx, seqlens


# "split": few heads, scores from a separate many-workgroup launch;
# "head": batch * kv heads >= 128, one workgroup per (b, kv head) end to end
# (the fused top-k step's scores come from a split scan first while batch * kv
# heads is below the CU count); "wide": batch * kv heads = 256, the fused
# top-k step scans in the same launch.
DECODE_SHAPES = {"split": (2, 2), "head": (8, 16), "wide": (8, 32)}


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("alpha", [1.5, 2.0])
@pytest.mark.parametrize("G", [1, 4])
@pytest.mark.parametrize("niter", [2, 10])
@pytest.mark.parametrize("path", ["split", "head"])
def test_decode_exact_matches_oracle(dtype, alpha, G, niter, path):
    K = _K()
    _case(test="decode_exact", dtype=dtype, alpha=alpha, G=G, niter=niter, path=path)
    rng = np.random.default_rng(100 + G)
    B, Hkv = DECODE_SHAPES[path]
    S, D = 16 * 200 + 3, 128
    Kc, Vc, q, pidx, seqlens = _decode_case(rng, dtype, B, Hkv, G, S, D, 64)
    H = Hkv * G
    dt = TORCH_DT[dtype]
    out = torch.zeros(B, H, 1, D, dtype=dt, device="cuda")
    taus = torch.zeros(B, H, dtype=torch.float32, device="cuda")
    K.sparse_attention_decode_paged(to_dev(q, dtype), to_dev(Kc, dtype), to_dev(Vc, dtype), out,
                                    torch.tensor(seqlens, dtype=torch.int32, device="cuda"),
                                    torch.tensor(pidx, dtype=torch.int32, device="cuda"), 16,
                                    alpha=alpha, niter=niter, taus_out=taus)
    torch.cuda.synchronize()
    ref, ref_tau = O.paged_entmax_decode(q[:, :, 0], Kc, Vc, pidx, seqlens, 16, alpha, niter, dtype)
    assert_out_close(to_np(out)[:, :, 0], ref, dtype)
    np.testing.assert_allclose(to_np(taus), ref_tau, atol=1e-4)
    if niter == 10 and path == "split":
        # converged: equals exact sort-based entmax over the selected tokens
        qs = O.scaled_query(q[:, :, 0], alpha, dtype)
        for b in range(B):
            for h in range(H):
                rows = O.compacted_rows(pidx[b, h // G], seqlens[b, h // G], 16)
                s = Kc[b, h // G][rows] @ qs[b, h]
                p = O.entmax_exact(s, alpha)
                assert_out_close(to_np(out)[b, h, 0], p @ Vc[b, h // G][rows], dtype, "exact")


@pytest.mark.parametrize("n_sel", [400, 1699])
def test_decode_long_heads(n_sel):
    """One workgroup per head with long selections: 6405 tokens (block-wide tau
    solve, scores staged in LDS) and 27189 tokens (scores in the workspace)."""
    K = _K()
    _case(test="decode_long", n_sel=n_sel)
    rng = np.random.default_rng(31)
    dtype = "fp16"
    B, Hkv, S, D = 1, 128, 16 * 1700 + 5, 32
    f16 = lambda *shape: rng.standard_normal(shape, dtype=np.float32).astype(np.float16).astype(np.float64)
    Kc, Vc, q = f16(B, Hkv, S, D), f16(B, Hkv, S, D), f16(B, Hkv, 1, D)
    P = (S + 15) // 16
    pidx = np.stack([np.stack([np.concatenate([np.sort(rng.permutation(P - 1)[:n_sel]), [P - 1]])
                               for _ in range(Hkv)]) for _ in range(B)])
    seqlens = np.full((B, Hkv), n_sel * 16 + S - (P - 1) * 16)
    out = torch.zeros(B, Hkv, 1, D, dtype=torch.float16, device="cuda")
    taus = torch.zeros(B, Hkv, dtype=torch.float32, device="cuda")
    K.sparse_attention_decode_paged(to_dev(q, dtype), to_dev(Kc, dtype), to_dev(Vc, dtype), out,
                                    torch.tensor(seqlens, dtype=torch.int32, device="cuda"),
                                    torch.tensor(pidx, dtype=torch.int32, device="cuda"), 16,
                                    alpha=1.5, niter=2, taus_out=taus)
    torch.cuda.synchronize()
    ref, ref_tau = O.paged_entmax_decode(q[:, :, 0], Kc, Vc, pidx, seqlens, 16, 1.5, 2, dtype)
    assert_out_close(to_np(out)[:, :, 0], ref, dtype)
    np.testing.assert_allclose(to_np(taus), ref_tau, atol=1e-4)


@pytest.mark.parametrize("dtype", ["fp16", "fp32"])
@pytest.mark.parametrize("iters", [0, 1, 2])
def test_decode_given_tau_matches_oracle(dtype, iters):
    K = _K()
    _case(test="decode_given_tau", dtype=dtype, iters=iters)
    rng = np.random.default_rng(7)
    B, Hkv, S, D = 2, 4, 16 * 100, 64
    Kc, Vc, q, pidx, seqlens = _decode_case(rng, dtype, B, Hkv, 1, S, D, 40)
    tau0 = O.paged_entmax_decode(q[:, :, 0], Kc, Vc, pidx, seqlens, 16, 1.5, 30, dtype)[1] - 0.05
    tau = torch.tensor(tau0, dtype=torch.float32, device="cuda").contiguous()
    out = torch.zeros(B, Hkv, 1, D, dtype=TORCH_DT[dtype], device="cuda")
    K.sparse_attention_decode_paged_gaussian_tau(
        to_dev(q, dtype), to_dev(Kc, dtype), to_dev(Vc, dtype), out,
        torch.tensor(seqlens, dtype=torch.int32, device="cuda"),
        torch.tensor(pidx, dtype=torch.int32, device="cuda"), 16, tau, alpha=1.5,
        tau_correction_iters=iters)
    torch.cuda.synchronize()
    ref, ref_tau = O.paged_entmax_decode(q[:, :, 0], Kc, Vc, pidx, seqlens, 16, 1.5, 0, dtype,
                                         tau_given=tau0, tau_iters=iters)
    assert_out_close(to_np(out)[:, :, 0], ref, dtype)
    np.testing.assert_allclose(to_np(tau), ref_tau, atol=1e-5)


def test_decode_edge_cases():
    """Empty and single-token heads, partial last page, out-of-range page ids."""
    K = _K()
    _case(test="decode_edges")
    rng = np.random.default_rng(9)
    dtype = "fp16"
    B, Hkv, S, D = 1, 4, 16 * 10 + 1, 128
    Kc = randn(rng, (B, Hkv, S, D), dtype)
    Vc = randn(rng, (B, Hkv, S, D), dtype)
    q = randn(rng, (B, Hkv, 1, D), dtype)
    pidx = np.array([[[3, 10, 0], [10, 0, 0], [2, 10, 0], [999999, 10, 0]]])
    seqlens = np.array([[17, 1, 0, 17]])
    out = torch.full((B, Hkv, 1, D), 7.0, dtype=torch.float16, device="cuda")
    K.sparse_attention_decode_paged(to_dev(q, dtype), to_dev(Kc, dtype), to_dev(Vc, dtype), out,
                                    torch.tensor(seqlens, dtype=torch.int32, device="cuda"),
                                    torch.tensor(pidx, dtype=torch.int32, device="cuda"), 16,
                                    alpha=1.5, niter=10)
    torch.cuda.synchronize()
    o = to_np(out)[0, :, 0]
    # head 1: a single token gets probability 1 -> out = v
    np.testing.assert_allclose(o[1], Vc[0, 1, 160], atol=2e-3)
    # head 2: no tokens -> zeros
    assert np.all(o[2] == 0)
    # head 0: page 3 + first row of page 10
    ref, _ = O.paged_entmax_decode(q[:, :1, 0], Kc[:, :1], Vc[:, :1], pidx[:, :1], seqlens[:, :1],
                                   16, 1.5, 10, dtype)
    assert_out_close(o[0], ref[0, 0], dtype)
    # head 3: the malformed page id is skipped, the last page still attends
    ref3, _ = O.paged_entmax_decode(q[:, 3:4, 0], Kc[:, 3:4], Vc[:, 3:4], np.array([[[10]]]),
                                    np.array([[1]]), 16, 1.5, 10, dtype)
    assert_out_close(o[3], ref3[0, 0], dtype)


# ---------------------------------------------------------------------------
# public top-k API end to end
# ---------------------------------------------------------------------------

# "split": few heads (criticality + top-k launch, then the decode launches);
# "head": one fused launch per step (criticality, top-k and decode per workgroup)
TOPK_API_CASES = [("fp16", 1, "split", False), ("bf16", 4, "split", False),
                  ("fp32", 1, "split", False), ("fp16", 1, "head", False),
                  ("bf16", 4, "head", False), ("fp32", 2, "head", False),
                  ("fp16", 1, "head", True), ("bf16", 8, "head", True),
                  ("fp16", 1, "wide", False), ("bf16", 4, "wide", True),
                  ("fp32", 2, "wide", False)]


@pytest.mark.parametrize("dtype,G,path,alibi", TOPK_API_CASES)
def test_topk_api_end_to_end(dtype, G, path, alibi):
    from entmaxkv_amd import sparse_attention_decode_paged
    _case(test="topk_api", dtype=dtype, G=G, path=path, alibi=alibi)
    rng = np.random.default_rng(21)
    B, Hkv = DECODE_SHAPES[path]
    S0, D, ps = 16 * 128, 128, 16
    H = Hkv * G
    cache, k, v = _build_cache(rng, B, Hkv, S0, D, dtype)
    q = randn(rng, (B, H, 1, D), dtype)
    kn = randn(rng, (B, Hkv, 1, D), dtype)
    vn = randn(rng, (B, Hkv, 1, D), dtype)
    slopes = np.exp2(-8.0 * np.arange(1, H + 1) / H).astype(np.float32) if alibi else None
    budget = 512
    S = S0 + 1
    P = (S + ps - 1) // ps
    n_sel = min(budget // ps, P - 1)
    lps = S - (P - 1) * ps
    out = torch.zeros(B, H, 1, D, dtype=TORCH_DT[dtype], device="cuda")
    sparse_attention_decode_paged(
        to_dev(q, dtype), cache, to_dev(kn, dtype), to_dev(vn, dtype), out, budget,
        torch.full((B,), n_sel * ps + lps, dtype=torch.int32, device="cuda"),
        torch.full((B,), S, dtype=torch.int32, device="cuda"),
        alibi_slopes=None if slopes is None else torch.tensor(slopes, device="cuda"),
        alpha=1.5, niter=10, append_cache=True)
    torch.cuda.synchronize()
    Kf = np.concatenate([k, kn], axis=2)
    Vf = np.concatenate([v, vn], axis=2)
    st = O.page_stats(Kf, ps, dtype)
    scores = to_np(cache.last_page_scores)
    ref_scores = O.page_criticality(q[:, :, 0], st[0], st[1], dtype, num_pages=P - 1,
                                    alibi_slopes=slopes, page_size=ps, seq_len=S, q_pos=S - 1)
    # fp32 accumulation order differs from the float64 oracle: bound on the
    # magnitudes summed (score terms and ALiBi bonus), then one rounding
    terms = np.abs(O.page_criticality(q[:, :, 0], st[0], st[1], "fp32", num_pages=P - 1))
    if slopes is not None:
        terms = terms + np.abs(O.alibi_page_bonus(slopes, P - 1, ps, S, S - 1))[None]
    ulp = {"fp16": 2.0 ** -10, "bf16": 2.0 ** -7, "fp32": 2.0 ** -23}[dtype]
    assert (np.abs(scores - ref_scores) <= 2.0 ** -20 * terms + ulp * np.abs(ref_scores)).all()
    # page table bit-exact given the kernel's scores
    sel = O.topk_gqa_pages(scores, Hkv, n_sel)
    pidx = np.concatenate([sel, np.full((B, Hkv, 1), P - 1)], axis=2)
    np.testing.assert_array_equal(to_np(cache._page_indices_buf).astype(np.int64), pidx)
    ref, _ = O.paged_entmax_decode(q[:, :, 0], Kf, Vf, pidx, np.full((B, Hkv), n_sel * ps + lps),
                                   ps, 1.5, 10, dtype, alibi_slopes=slopes, q_seqlens=np.full(B, S))
    assert_out_close(to_np(out)[:, :, 0], ref, dtype)


def test_config1_topk_step():
    """benchmark config 1 on the GPU: B=1, H=32, D=128, 1024-token prefill + one
    appended token, page size 16, fp32, budget 256, alpha 1.5 (niter 10): the
    page table equals the oracle's top-k of the kernel's scores and the output
    equals the oracle step within 1e-5."""
    from entmaxkv_amd import sparse_attention_decode_paged
    _case(test="config1")
    rng = np.random.default_rng(0)
    B, H, S0, D, ps, budget, dtype = 1, 32, 1024, 128, 16, 256, "fp32"
    cache, k, v = _build_cache(rng, B, H, S0, D, dtype)
    q = randn(rng, (B, H, 1, D), dtype)
    kn = randn(rng, (B, H, 1, D), dtype)
    vn = randn(rng, (B, H, 1, D), dtype)
    S = S0 + 1
    P = (S + ps - 1) // ps
    n_sel = budget // ps
    out = torch.zeros(B, H, 1, D, dtype=torch.float32, device="cuda")
    sparse_attention_decode_paged(
        to_dev(q, dtype), cache, to_dev(kn, dtype), to_dev(vn, dtype), out, budget,
        torch.full((B,), n_sel * ps + 1, dtype=torch.int32, device="cuda"),
        torch.full((B,), S, dtype=torch.int32, device="cuda"), alpha=1.5, niter=10)
    torch.cuda.synchronize()
    Kf = np.concatenate([k, kn], axis=2)
    Vf = np.concatenate([v, vn], axis=2)
    scores = to_np(cache.last_page_scores)
    pidx = np.concatenate([O.topk_pages(scores, n_sel), np.full((B, H, 1), P - 1)], axis=2)
    np.testing.assert_array_equal(to_np(cache._page_indices_buf).astype(np.int64), pidx)
    ref, _ = O.paged_entmax_decode(q[:, :, 0], Kf, Vf, pidx, np.full((B, H), n_sel * ps + 1), ps,
                                   1.5, 10, dtype)
    assert_out_close(to_np(out)[:, :, 0], ref, dtype)


@pytest.mark.parametrize("path,niter", [("head", 2), ("head", 10), ("split", 10)])
def test_config4_topk_step(path, niter):
    """benchmark config 4's top-k step at a shorter length: 32 query / 8 kv
    heads (G = 4), D = 128, bf16, alpha = 2 (sparsemax), budget 2048 tokens
    (128 pages + the last page per kv head), one appended token, q/k/v ~ N(0, 1).
    "head": B = 16 as in the config (one fused launch per step, prescored);
    "split": B = 2, Hkv = 2.  The reference cannot run GQA (its decode asserts
    one page table per query head, adadecode_paged.py:600), so the oracle's
    best-rank GQA table and exact-tau decode are the reference."""
    from entmaxkv_amd import sparse_attention_decode_paged
    _case(test="config4_topk", path=path, niter=niter)
    rng = np.random.default_rng(4)
    dtype, G, alpha, ps, D, budget = "bf16", 4, 2.0, 16, 128, 2048
    B, Hkv = (16, 8) if path == "head" else (2, 2)
    S0 = 16 * 200
    H = Hkv * G
    cache, k, v = _build_cache(rng, B, Hkv, S0, D, dtype)
    q = randn(rng, (B, H, 1, D), dtype)
    kn = randn(rng, (B, Hkv, 1, D), dtype)
    vn = randn(rng, (B, Hkv, 1, D), dtype)
    S = S0 + 1
    P = (S + ps - 1) // ps
    n_sel = min(budget // ps, P - 1)
    lps = S - (P - 1) * ps
    out = torch.zeros(B, H, 1, D, dtype=TORCH_DT[dtype], device="cuda")
    sparse_attention_decode_paged(
        to_dev(q, dtype), cache, to_dev(kn, dtype), to_dev(vn, dtype), out, budget,
        torch.full((B,), n_sel * ps + lps, dtype=torch.int32, device="cuda"),
        torch.full((B,), S, dtype=torch.int32, device="cuda"), alpha=alpha, niter=niter,
        append_cache=True)
    torch.cuda.synchronize()
    Kf = np.concatenate([k, kn], axis=2)
    Vf = np.concatenate([v, vn], axis=2)
    st = O.page_stats(Kf, ps, dtype)
    scores = to_np(cache.last_page_scores)
    ref_scores = O.page_criticality(q[:, :, 0], st[0], st[1], dtype, num_pages=P - 1)
    terms = np.abs(O.page_criticality(q[:, :, 0], st[0], st[1], "fp32", num_pages=P - 1))
    assert (np.abs(scores - ref_scores) <= 2.0 ** -20 * terms + 2.0 ** -7 * np.abs(ref_scores)).all()
    sel = O.topk_gqa_pages(scores, Hkv, n_sel)
    pidx = np.concatenate([sel, np.full((B, Hkv, 1), P - 1)], axis=2)
    np.testing.assert_array_equal(to_np(cache._page_indices_buf).astype(np.int64), pidx)
    ref, _ = O.paged_entmax_decode(q[:, :, 0], Kf, Vf, pidx, np.full((B, Hkv), n_sel * ps + lps),
                                   ps, alpha, niter, dtype)
    assert_out_close(to_np(out)[:, :, 0], ref, dtype)


# ---------------------------------------------------------------------------
# a7 - a12 Gaussian path
# ---------------------------------------------------------------------------

def _gaussian_inputs(rng, dtype, B, H, S, D, outlier_frac=0.0):
    k = rng.standard_normal((B, H, S, D)) + rng.standard_normal((B, H, 1, 1)) * math.sqrt(0.5)
    q = rng.standard_normal((B, H, 1, D))
    if outlier_frac:
        P = S // 16
        for b in range(B):
            for h in range(H):
                pages = rng.choice(P, max(1, int(outlier_frac * P)), replace=False)
                for p in pages:
                    qh = q[b, h, 0] / np.linalg.norm(q[b, h, 0])
                    k[b, h, p * 16:(p + 1) * 16] = 3.0 * (k[b, h, p * 16:(p + 1) * 16] + 4.0 * qh)
    return O.round_to(q, dtype), O.round_to(k, dtype), randn(rng, (B, H, S, D), dtype)


@pytest.mark.parametrize("dtype", ["fp16", "fp32"])
@pytest.mark.parametrize("alpha", [1.5, 2.0])
def test_gaussian_stats_tau_select_clamp(dtype, alpha):
    K = _K()
    from entmaxkv_amd import PagedKVCache
    from entmaxkv_amd.gaussian_utils import compute_gaussian_aware_statistics
    _case(test="gaussian_pipeline", dtype=dtype, alpha=alpha)
    rng = np.random.default_rng(31)
    B, H, S, D, ps = 2, 4, 16 * 256 + 1, 128, 16
    q, k, v = _gaussian_inputs(rng, dtype, B, H, S, D, outlier_frac=0.02)
    cache = PagedKVCache(page_size=ps)
    cache.initialize(to_dev(k, dtype), to_dev(v, dtype))
    qd = to_dev(q, dtype)
    st = compute_gaussian_aware_statistics(qd, cache.k_mean, cache.k_std, S, ps, alpha=alpha,
                                           buffers=cache.get_gaussian_buffers(qd, cache.num_pages - 1))
    lps = O.last_page_size(S, ps)
    pidx, counts = cache.select_gaussian_aware(qd, alpha=alpha, gaussian_stats=st, clamp=True,
                                               last_page_size=lps)
    torch.cuda.synchronize()
    P = cache.num_pages
    pfs = P - 1
    # the kernel is checked on the statistics the cache holds (those are pinned
    # separately by test_page_stats_initialize)
    ref = O.gaussian_page_stats(q[:, :, 0], to_np(cache.k_mean), to_np(cache.k_std), pfs)
    mu_p, sg_p = to_np(st["mu_scores_per_page"]), to_np(st["sigma_scores_per_page"])
    np.testing.assert_allclose(mu_p, ref["mu_p"], rtol=1e-5, atol=1e-5)
    np.testing.assert_allclose(sg_p, ref["sigma_p"], rtol=1e-5, atol=1e-6)
    sg_g = to_np(st["sigma_global"])[..., 0]
    mu_g = to_np(st["mu_global"])[..., 0]
    np.testing.assert_allclose(mu_g, ref["mu_g"], rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(sg_g, ref["sigma_g"], rtol=1e-5)
    # tau-hat from the GPU's own global moments
    th = to_np(st["tau_hat"])
    ref_th = O.tau_single_gaussian(mu_g, sg_g, pfs * ps, alpha)
    np.testing.assert_allclose(th, ref_th, atol=2e-5, rtol=2e-5)
    # auto margins, tau floor
    smz, mq = O.auto_selection_margins(sg_g)
    eff = to_np(st["effective_margins"])
    np.testing.assert_allclose(eff, [smz, mq], rtol=1e-5)
    tf = to_np(st["tau_floor"])
    ref_tf = O.tau_floor_fp32(mu_p, sg_p, th, sg_g, alpha, np.float32(eff[0]), 0.2, pfs)
    np.testing.assert_allclose(tf, ref_tf, atol=1e-5, rtol=1e-5)
    # selection: bit-exact given the GPU's moments and floor
    z_page = O.page_quantile_z(0.995 if eff[1] > 0.992 else 0.99, ps)
    packed, ref_counts = O.select_gaussian_pages(mu_p, sg_p, tf, alpha, z_page, pfs, P)
    got_pidx = to_np(pidx).astype(np.int64)
    got_counts = to_np(counts).astype(np.int64)
    np.testing.assert_array_equal(got_counts, ref_counts)
    for b in range(B):
        for h in range(H):
            np.testing.assert_array_equal(got_pidx[b, h, :got_counts[b, h]], packed[b, h])
    np.testing.assert_array_equal(to_np(st["cache_seqlens"]),
                                  O.cache_seqlens_from_counts(ref_counts, ps, lps))
    ref_tc = O.tau_clamp(th, mu_p, sg_p, packed, ref_counts, tf, alpha,
                         O.page_quantile_z(0.5, ps), pfs)
    np.testing.assert_allclose(to_np(st["tau_clamped"]), ref_tc, atol=1e-6, rtol=1e-6)
    # standalone clamp entry point agrees with the fused one
    tc2 = K.clamp_tau_to_selected_page_statistics(st["tau_hat"], st["mu_scores_per_page"],
                                                   st["sigma_scores_per_page"], pidx, counts,
                                                   st["tau_floor"], ps, alpha, 0.5, pfs)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(to_np(tc2), to_np(st["tau_clamped"]))


@pytest.mark.parametrize("tau_mode", ["exact", "fixed", "corrected"])
def test_gaussian_api_end_to_end(tau_mode):
    from entmaxkv_amd import PagedKVCache, sparse_attention_decode_gaussian_aware_entmax
    _case(test="gaussian_api", tau_mode=tau_mode)
    dtype = "fp16"
    rng = np.random.default_rng(41)
    B, H, S, D, ps = 2, 4, 16 * 128 + 1, 128, 16
    q, k, v = _gaussian_inputs(rng, dtype, B, H, S, D, outlier_frac=0.02)
    cache = PagedKVCache(page_size=ps)
    cache.initialize(to_dev(k, dtype), to_dev(v, dtype))
    out = torch.zeros(B, H, 1, D, dtype=torch.float16, device="cuda")
    sparse_attention_decode_gaussian_aware_entmax(to_dev(q, dtype), cache, None, None, out,
                                                  alpha=1.5, tau_mode=tau_mode)
    torch.cuda.synchronize()
    _check_gaussian_step(cache, q, k, v, out, dtype, 1, tau_mode, 1.5, [S] * B)


@pytest.mark.parametrize("pages", [4000, 4200])
def test_gaussian_moments_store_branches(pages):
    """moments_kernel stages mu_p, sigma_p in LDS while a workgroup's pages times
    the group fit 4096 entries, else stores them from the scan loop.  G = 8 with
    B * Hkv = 128 splits each head into 8 workgroups: 4000 pages stay under the
    limit (500 * 8), 4200 go over it (525 * 8)."""
    K = _K()
    _case(test="gaussian_moments_branches", pages=pages)
    rng = np.random.default_rng(pages)
    dtype, B, Hkv, G, D = "fp16", 8, 16, 8, 64
    H = Hkv * G
    q = randn(rng, (B, H, 1, D), dtype)
    km = randn(rng, (B, Hkv, pages + 1, D), dtype, 0.5)
    ks = O.round_to(np.abs(rng.standard_normal((B, Hkv, pages + 1, D))) * 0.5 + 0.05, dtype)
    buf = K.compute_page_gaussian_stats(to_dev(q, dtype), to_dev(km, dtype), to_dev(ks, dtype),
                                        pages, page_size=16, seq_len=16 * pages + 1,
                                        solve_tau=False)
    torch.cuda.synchronize()
    ref = O.gaussian_page_stats(q[:, :, 0], km, ks, pages)
    np.testing.assert_allclose(to_np(buf.mu_p), ref["mu_p"], rtol=1e-5, atol=1e-5)
    np.testing.assert_allclose(to_np(buf.sigma_p), ref["sigma_p"], rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(to_np(buf.mu_g)[..., 0], ref["mu_g"], rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(to_np(buf.sigma_g)[..., 0], ref["sigma_g"], rtol=1e-5)


def test_tau_mixture_matches_oracle():
    K = _K()
    _case(test="tau_mixture")
    rng = np.random.default_rng(51)
    mu = rng.standard_normal((3, 200)).astype(np.float32)
    sg = (np.abs(rng.standard_normal((3, 200))) + 0.1).astype(np.float32)
    for alpha in (1.5, 2.0):
        got = K.solve_for_tau_hat_page_gaussian_mixture(torch.tensor(mu, device="cuda"),
                                                        torch.tensor(sg, device="cuda"),
                                                        alpha=alpha, uniform_page_count=16.0)
        torch.cuda.synchronize()
        ref = O.tau_page_mixture(mu, sg, 16.0, alpha)
        np.testing.assert_allclose(to_np(got)[:, 0], ref, atol=5e-5, rtol=5e-5)


def test_tau_single_matches_oracle():
    K = _K()
    _case(test="tau_single")
    mu = np.array([0.1, -0.5, 0.0, 2.0, 0.3], np.float32)
    sg = np.array([0.3, 1.2, 0.05, 0.7, 2.5], np.float32)
    for alpha in (1.5, 2.0):
        for n in (16, 2048, 32768):
            got = K.solve_for_tau_hat_single_gaussian_gpu(torch.tensor(mu, device="cuda"),
                                                          torch.tensor(sg, device="cuda"), n, alpha)
            torch.cuda.synchronize()
            ref = O.tau_single_gaussian(mu, sg, n, alpha)
            np.testing.assert_allclose(to_np(got), ref, atol=2e-5, rtol=2e-5)


def _gqa_gaussian_inputs(rng, dtype, B, Hkv, G, S, D, outlier_frac):
    """Keys ~ N(mu_h, 1) per kv head with a fraction of pages scaled x3 and pulled
    toward the group's first query head; q, v ~ N(0, 1)."""
    H = Hkv * G
    k = rng.standard_normal((B, Hkv, S, D)) + rng.standard_normal((B, Hkv, 1, 1)) * math.sqrt(0.5)
    q = rng.standard_normal((B, H, 1, D))
    P = S // 16
    n_out = max(1, int(outlier_frac * P))
    for b in range(B):
        for kvh in range(Hkv):
            qh = q[b, kvh * G, 0] / np.linalg.norm(q[b, kvh * G, 0])
            for p in rng.choice(P, n_out, replace=False):
                k[b, kvh, p * 16:(p + 1) * 16] = 3.0 * (k[b, kvh, p * 16:(p + 1) * 16] + 4.0 * qh)
    return O.round_to(q, dtype), O.round_to(k, dtype), randn(rng, (B, Hkv, S, D), dtype)


# (dtype, G, tau_mode, alpha, B, Hkv, D, keys).  B * Hkv >= 128 runs one fused
# launch per step, B * Hkv = 4 the split launches.  The D = 128 rows are the
# shapes the benchmark times: the headline Gaussian step (fp16, G = 1, B * Hkv
# = 256) and config 4 (bf16, 32 q / 8 kv heads, alpha = 2, B = 16, N(0, 1)
# keys), at a shorter length.
GAUSS_FUSED_CASES = [("fp16", 1, "corrected", 1.5, 8, 16, 64, "c3"),
                     ("bf16", 1, "exact", 1.5, 8, 16, 64, "c3"),
                     ("fp32", 1, "fixed", 2.0, 8, 16, 64, "c3"),
                     ("fp16", 4, "corrected", 1.5, 8, 16, 64, "c3"),
                     ("bf16", 2, "corrected", 2.0, 8, 16, 64, "c3"),
                     ("fp16", 8, "exact", 1.5, 8, 16, 64, "c3"),
                     ("fp16", 1, "corrected", 1.5, 8, 32, 128, "c3"),
                     ("bf16", 4, "corrected", 2.0, 16, 8, 128, "iid"),
                     ("bf16", 4, "exact", 2.0, 16, 8, 128, "iid"),
                     ("bf16", 4, "corrected", 2.0, 2, 2, 128, "iid"),
                     ("bf16", 4, "fixed", 2.0, 2, 2, 128, "c3")]


def _check_gaussian_step(cache, q, k, v, out, dtype, G, tau_mode, alpha, lens, slopes=None):
    """The Gaussian step's stages against the oracle, sequence by sequence.

    ``lens`` [B]: the sequence lengths (all equal for a uniform batch).  The
    automatic margins are batch-wide, so they come from every head's sigma_g;
    everything else is per sequence.  With ALiBi ``slopes`` [H] the page means
    carry the page-mean bias, tau-hat is the page-mixture root and the decode
    adds the position bias at q position lens[b] - 1 (the step is run with
    q_seqlens = lens)."""
    st = cache.last_gaussian_stats
    ps = cache.page_size
    B, H = q.shape[:2]
    Hkv = H // G
    mu_p_all, sg_p_all = to_np(st["mu_scores_per_page"]), to_np(st["sigma_scores_per_page"])
    mu_g = to_np(st["mu_global"])[..., 0]
    sg_g = to_np(st["sigma_global"])[..., 0]
    th = to_np(st["tau_hat"])
    tf = to_np(st["tau_floor"])
    eff = to_np(st["effective_margins"])
    smz, mq = O.auto_selection_margins(sg_g)
    np.testing.assert_allclose(eff, [smz, mq], rtol=1e-5)
    z_page = O.page_quantile_z(0.995 if eff[1] > 0.992 else 0.99, ps)
    counts = to_np(cache.last_num_selected_per_head).astype(np.int64)
    pidx_all = to_np(cache._select_buffers[next(iter(cache._select_buffers))]["page_indices"]).astype(np.int64)
    seqlens_got = to_np(st["cache_seqlens"]).astype(np.int64)
    tau_cl = to_np(st["tau_clamped"]) if tau_mode != "exact" else None
    tau_fin = to_np(st["tau_final"]) if tau_mode != "exact" else None
    got_out = to_np(out)[:, :, 0]
    kmean_all, kstd_all = to_np(cache.k_mean), to_np(cache.k_std)
    stats = {"rows": 0, "ambiguous_rows": 0}
    for b in range(B):
        S = int(lens[b])
        P = (S + ps - 1) // ps
        pfs = P - 1 if P > 1 else P
        n_stats = pfs * ps if P > 1 else S
        lps = O.last_page_size(S, ps)
        sl = slice(b, b + 1)
        ref = O.gaussian_page_stats(q[sl, :, 0], kmean_all[sl, :, :P], kstd_all[sl, :, :P], pfs)
        mu_p, sg_p = mu_p_all[sl, :, :pfs], sg_p_all[sl, :, :pfs]
        ref_mu = ref["mu_p"]
        if slopes is not None:
            ref_mu = ref_mu + O.alibi_page_mean_bias(slopes, pfs, S, ps)[None]
        np.testing.assert_allclose(mu_p, ref_mu, rtol=1e-5, atol=1e-5)
        np.testing.assert_allclose(sg_p, ref["sigma_p"], rtol=1e-5, atol=1e-6)
        np.testing.assert_allclose(mu_g[sl], ref["mu_g"], rtol=1e-5, atol=1e-6)
        np.testing.assert_allclose(sg_g[sl], ref["sigma_g"], rtol=1e-5)
        if slopes is None:
            ref_th = O.tau_single_gaussian(mu_g[sl], sg_g[sl], n_stats, alpha)
        else:
            ref_th = O.tau_page_mixture(mu_p, sg_p, float(ps), alpha)
        np.testing.assert_allclose(th[sl], ref_th, atol=5e-5, rtol=2e-5)
        np.testing.assert_allclose(tf[sl], O.tau_floor_fp32(mu_p, sg_p, th[sl], sg_g[sl], alpha,
                                                            np.float32(eff[0]), 0.2, pfs),
                                   atol=1e-5, rtol=1e-5)
        # page table: the union over each kv head's query heads, bit-exact given
        # the kernel's moments and floor
        packed_q, _ = O.select_gaussian_pages(mu_p, sg_p, tf[sl], alpha, z_page, pfs, P)
        pidx = np.zeros((1, Hkv, max(P, 1)), dtype=np.int64)
        packed_rows = np.empty((1, H), dtype=object)
        for kvh in range(Hkv):
            u = np.unique(np.concatenate([packed_q[0, kvh * G + g] for g in range(G)]))
            assert counts[b, kvh] == u.size
            np.testing.assert_array_equal(pidx_all[b, kvh, :u.size], u)
            pidx[0, kvh, :u.size] = u
            for g in range(G):
                packed_rows[0, kvh * G + g] = u
        seqlens = O.cache_seqlens_from_counts(counts[sl], ps, lps)
        np.testing.assert_array_equal(seqlens_got[sl], seqlens)
        kb, vb = k[sl, :, :S], v[sl, :, :S]
        ali = {} if slopes is None else {"alibi_slopes": slopes, "q_seqlens": np.array([S])}
        if tau_mode == "exact":
            ref_out, _ = O.paged_entmax_decode(q[sl, :, 0], kb, vb, pidx, seqlens, ps, alpha, 2,
                                               dtype, **ali)
            assert_out_close(got_out[sl], ref_out, dtype)
            continue
        tc = O.tau_clamp(th[sl], mu_p, sg_p, packed_rows, np.repeat(counts[sl], G, axis=1), tf[sl],
                         alpha, O.page_quantile_z(0.5, ps), pfs)
        np.testing.assert_allclose(tau_cl[sl], tc, atol=1e-6, rtol=1e-6)
        iters = 0 if tau_mode == "fixed" else (1 if slopes is None else 2)
        tau_in = tau_cl[sl]
        ref_out, ref_tau = O.paged_entmax_decode(q[sl, :, 0], kb, vb, pidx, seqlens, ps, alpha, 0,
                                                 dtype, tau_given=tau_in, tau_iters=iters, **ali)
        # The corrected tau (adadecode_paged_gaussian_tau.py:12-53).  A score within
        # its own fp32 rounding of tau_in can land on either side of tau_in in the
        # kernel; that moves it in or out of the support the Halley step sums over
        # (for alpha = 1.5 the support count is f'').  Such a row gets two more
        # oracle references, its ambiguous scores all inside or all outside the
        # support, and the kernel must match one of them.  No row is exempt.
        qs = O.scaled_query(q[sl, :, 0], alpha, dtype)
        tf_b = tau_fin[sl]
        tau_ref = np.array(ref_tau, dtype=np.float64)
        cond = np.ones((1, H))
        mass = np.ones((1, H, 1))
        for h in range(H):
            rows = O.compacted_rows(pidx[0, h // G], seqlens[0, h // G], ps)
            kr = np.asarray(kb[0, h // G], np.float64)[rows]
            sc = O.head_scores(qs[0, h], kb[0, h // G], rows,
                               0.0 if slopes is None else float(slopes[h]), alpha, S - 1)
            if not iters:
                mass[0, h, 0] = max(1.0, O.entmax_weights(sc, tau_ref[0, h], alpha).sum())
                continue
            t_in = float(tau_in[0, h])
            eps = 2.0 ** -20 * (np.abs(kr) @ np.abs(qs[0, h]) + np.abs(sc))
            amb = np.abs(sc - t_in) <= eps
            cands = [float(ref_tau[0, h])]
            if amb.any():
                stats["ambiguous_rows"] += 1
                for inside in (True, False):
                    t = _corrected_step_with_support(sc, t_in, amb, inside, alpha)
                    for _ in range(iters - 1):
                        t = O.halley_unbounded_update(t, *O.entmax_accumulators(sc, t, alpha),
                                                      alpha)
                    cands.append(t)
            tau_ref[0, h] = min(cands, key=lambda t: abs(t - float(tf_b[0, h])))
            # condition of the step: 2 f'^2 - f f'' can nearly cancel, and the step
            # then amplifies the fp32 rounding of the kernel's accumulators by
            # (2 f'^2 + |f f''|) / |2 f'^2 - f f''|
            a0, a1, a2 = O.entmax_accumulators(sc, t_in, alpha)
            c0 = 1.0 / (alpha - 1.0)
            f, df, ddf = a0 - 1.0, -c0 * a1, c0 * (c0 - 1.0) * a2
            den = abs(2 * df * df - f * ddf)
            cond[0, h] = (2 * df * df + abs(f * ddf)) / den if den > 0 else np.inf
            mass[0, h, 0] = max(1.0, O.entmax_weights(sc, tau_ref[0, h], alpha).sum())
        stats["rows"] += H
        # fp32 accumulators carry a relative error of about 1e-6; the bar allows
        # ten times that, amplified by the step's condition
        with np.errstate(invalid="ignore"):
            amp = np.nan_to_num(np.abs(tau_ref - tau_in) * cond, nan=0.0)
        tol = 1e-4 + 1e-5 * np.abs(tau_ref) + 1e-5 * amp
        bad = np.abs(tf_b - tau_ref) > tol
        assert not bad.any(), (f"tau_final: {bad.sum()} rows beyond tolerance, worst "
                               f"{np.abs(tf_b - tau_ref)[bad].max():.3g}")
        ref_out, _ = O.paged_entmax_decode(q[sl, :, 0], kb, vb, pidx, seqlens, ps, alpha, 0,
                                           dtype, tau_given=tau_ref, tau_iters=0, **ali)
        # the weighted sum at the kernel's own final tau
        ref_at_fin, _ = O.paged_entmax_decode(q[sl, :, 0], kb, vb, pidx, seqlens, ps, alpha, 0,
                                              dtype, tau_given=tf_b, tau_iters=0, **ali)
        # given tau, out = sum_i [s_i - tau]_+^(1/(alpha-1)) v_i is not normalised:
        # its weights sum to `mass`, not 1, so outputs are compared divided by
        # max(1, mass), the normalised attention output, at the 2e-3 bar
        got = got_out[sl]
        # an un-normalised sum beyond the storage range is stored as +-inf
        big = np.abs(ref_at_fin) > {"fp16": 65504.0, "bf16": 3.3e38, "fp32": 3.4e38}[dtype]
        assert (np.isinf(got[big]) & (np.sign(got[big]) == np.sign(ref_at_fin[big]))).all()
        got = np.where(big, 0.0, got)
        assert_out_close(got / mass, np.where(big, 0.0, ref_at_fin) / mass, dtype)
        assert_out_close((got / mass)[~big], (ref_out / mass)[~big], dtype)
    if stats["rows"]:
        print(f"corrected tau: {stats['ambiguous_rows']} of {stats['rows']} rows had a score "
              f"within fp32 rounding of tau_in (checked against both support choices)",
              flush=True)
    return stats


def _corrected_step_with_support(sc, t_in, amb, inside, alpha):
    """One unbounded Halley step from t_in (the oracle's update) with the
    ambiguous scores ``amb`` forced inside or outside the support."""
    a = sc - t_in
    m = ((a > 0) & ~amb) | (amb & inside)
    am = a[m]
    if alpha == 2.0:
        acc = (float(np.sum(am)), float(m.sum()), 0.0)
    elif alpha == 1.5:
        acc = (float(np.sum(am * am)), float(np.sum(am)), float(m.sum()))
    else:
        c0 = 1.0 / (alpha - 1.0)
        am = np.maximum(am, 0.0)
        acc = (float(np.sum(am ** c0)), float(np.sum(am ** (c0 - 1))), float(np.sum(am ** (c0 - 2))))
    return O.halley_unbounded_update(t_in, *acc, alpha)


@pytest.mark.parametrize("dtype,G,tau_mode,alpha,B,Hkv,D,keys", GAUSS_FUSED_CASES)
def test_gaussian_fused_step(dtype, G, tau_mode, alpha, B, Hkv, D, keys):
    """The Gaussian step (global moments, tau-hat, selection, clamp and decode;
    one launch per step when B * Hkv >= 128) against the oracle, stage by stage."""
    from entmaxkv_amd import PagedKVCache, sparse_attention_decode_gaussian_aware_entmax
    _case(test="gaussian_fused", dtype=dtype, G=G, tau_mode=tau_mode, alpha=alpha, B=B, Hkv=Hkv,
          D=D, keys=keys)
    rng = np.random.default_rng(61 + G + D)
    S, ps = 16 * 96 + 5, 16
    H = Hkv * G
    if keys == "c3":
        q, k, v = _gqa_gaussian_inputs(rng, dtype, B, Hkv, G, S, D, 0.03)
    else:
        q, k, v = (randn(rng, (B, H, 1, D), dtype), randn(rng, (B, Hkv, S, D), dtype),
                   randn(rng, (B, Hkv, S, D), dtype))
    cache = PagedKVCache(page_size=ps)
    cache.initialize(to_dev(k, dtype), to_dev(v, dtype))
    out = torch.zeros(B, H, 1, D, dtype=TORCH_DT[dtype], device="cuda")
    sparse_attention_decode_gaussian_aware_entmax(to_dev(q, dtype), cache, None, None, out,
                                                  alpha=alpha, tau_mode=tau_mode)
    torch.cuda.synchronize()
    _check_gaussian_step(cache, q, k, v, out, dtype, G, tau_mode, alpha, [S] * B)


@pytest.mark.parametrize("tau_mode", ["corrected", "exact"])
def test_gaussian_paired_decode(tau_mode):
    """Groups of 4 at B * Hkv = 128 run the paired Gaussian launch: two
    workgroups per (b, kv head) select the same pages, and from 8192 selected
    tokens on each scores half of them and the later one, after a hand-off of
    its partner's scores, solves tau and gathers V.  N(0, 1) keys select about
    57 % of 1024 pages here (about 9300 tokens), so the hand-off runs; the
    step is checked against the oracle like any other."""
    from entmaxkv_amd import PagedKVCache, sparse_attention_decode_gaussian_aware_entmax
    dtype, G, alpha, B, Hkv, D = "bf16", 4, 2.0, 16, 8, 64
    _case(test="gaussian_paired", tau_mode=tau_mode, B=B, Hkv=Hkv, G=G, D=D)
    rng = np.random.default_rng(640)
    S, ps = 16 * 1024 + 5, 16
    H = Hkv * G
    q, k, v = (randn(rng, (B, H, 1, D), dtype), randn(rng, (B, Hkv, S, D), dtype),
               randn(rng, (B, Hkv, S, D), dtype))
    cache = PagedKVCache(page_size=ps)
    cache.initialize(to_dev(k, dtype), to_dev(v, dtype))
    out = torch.zeros(B, H, 1, D, dtype=TORCH_DT[dtype], device="cuda")
    sparse_attention_decode_gaussian_aware_entmax(to_dev(q, dtype), cache, None, None, out,
                                                  alpha=alpha, tau_mode=tau_mode)
    torch.cuda.synchronize()
    sel = cache.last_num_selected_per_head
    assert int(sel.min()) * ps >= 8192, "the selection is too small to take the hand-off"
    _check_gaussian_step(cache, q, k, v, out, dtype, G, tau_mode, alpha, [S] * B)


@pytest.mark.parametrize("path", ["head", "split"])
def test_gaussian_alibi_step(path):
    """ALiBi through the Gaussian step: page-mean bias on the page means,
    page-mixture tau-hat given to the fused launch, two corrections and the
    position bias in the decode (attention_gaussian.py:103-140,
    gaussian_utils.py:142-181)."""
    from entmaxkv_amd import PagedKVCache, sparse_attention_decode_gaussian_aware_entmax
    _case(test="gaussian_alibi", path=path)
    dtype, alpha, G = "fp16", 1.5, 2
    rng = np.random.default_rng(91)
    B, Hkv = (8, 16) if path == "head" else (2, 2)
    S, D, ps = 16 * 64 + 7, 64, 16
    H = Hkv * G
    q, k, v = _gqa_gaussian_inputs(rng, dtype, B, Hkv, G, S, D, 0.03)
    slopes = np.exp2(-8.0 * np.arange(1, H + 1) / H).astype(np.float32)
    cache = PagedKVCache(page_size=ps)
    cache.initialize(to_dev(k, dtype), to_dev(v, dtype))
    out = torch.zeros(B, H, 1, D, dtype=TORCH_DT[dtype], device="cuda")
    sparse_attention_decode_gaussian_aware_entmax(
        to_dev(q, dtype), cache, None, None, out, alpha=alpha, tau_mode="corrected",
        alibi_slopes=torch.tensor(slopes, device="cuda"),
        q_seqlens=torch.full((B,), S, dtype=torch.int32, device="cuda"))
    torch.cuda.synchronize()
    _check_gaussian_step(cache, q, k, v, out, dtype, G, "corrected", alpha, [S] * B,
                         slopes=slopes.astype(np.float64))


@pytest.mark.parametrize("shape", [(1, 1), (16, 8)])
def test_topk_gqa_sequential_candidate_lists(shape):
    """G = 8 with k = 2048 of 4096 pages: the group's candidate lists do not
    fit LDS together, so the heads' selects run one after another (the split
    top-k kernel for B * Hkv = 1; the one-workgroup-per-head criticality
    kernel for 128, whose fused step does not fit one workgroup)."""
    from entmaxkv_amd import sparse_attention_decode_paged
    B, Hkv = shape
    G, ps, D, dtype = 8, 16, 128, "bf16"
    _case(test="topk_gqa_sequential", B=B, Hkv=Hkv, G=G)
    rng = np.random.default_rng(77)
    S0 = 16 * 4096
    H = Hkv * G
    cache, k, v = _build_cache(rng, B, Hkv, S0, D, dtype)
    q = randn(rng, (B, H, 1, D), dtype)
    kn = randn(rng, (B, Hkv, 1, D), dtype)
    vn = randn(rng, (B, Hkv, 1, D), dtype)
    S = S0 + 1
    P = (S + ps - 1) // ps
    budget = 2048 * ps
    n_sel = min(budget // ps, P - 1)
    out = torch.zeros(B, H, 1, D, dtype=TORCH_DT[dtype], device="cuda")
    sparse_attention_decode_paged(
        to_dev(q, dtype), cache, to_dev(kn, dtype), to_dev(vn, dtype), out, budget,
        torch.full((B,), n_sel * ps + 1, dtype=torch.int32, device="cuda"),
        torch.full((B,), S, dtype=torch.int32, device="cuda"), alpha=1.5, niter=10,
        append_cache=True)
    torch.cuda.synchronize()
    sel = O.topk_gqa_pages(to_np(cache.last_page_scores), Hkv, n_sel)
    pidx = np.concatenate([sel, np.full((B, Hkv, 1), P - 1)], axis=2)
    np.testing.assert_array_equal(to_np(cache._page_indices_buf).astype(np.int64), pidx)
    if B * Hkv == 1:
        Kf = np.concatenate([k, kn], axis=2)
        Vf = np.concatenate([v, vn], axis=2)
        ref, _ = O.paged_entmax_decode(q[:, :, 0], Kf, Vf, pidx, np.full((B, Hkv), n_sel * ps + 1),
                                       ps, 1.5, 10, dtype)
        assert_out_close(to_np(out)[:, :, 0], ref, dtype)
