"""CPU oracle for the sparse-entmax paged decode path (TEST INFRASTRUCTURE ONLY).

This module is the checker, never the product: only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
import it.  The product path (``entmaxkv_amd``) never routes through it and
raises when its HIP library is missing.

It restates the reference algorithm in NumPy, in float64 unless a function
says otherwise.  Every function cites the reference file:line it follows
(paths relative to the deep-spin/entmaxkv repository root).  The reference
itself is Triton + PyTorch and cannot run here (no CUDA GPU); nothing from it
is imported.

Rounding points that the oracle reproduces on purpose:
  * the decode query is scaled by (alpha-1)/sqrt(D) in the input dtype
    (constant and product rounded to it, kernels/adadecode_paged.py:97-98);
  * page statistics and criticality scores are rounded to the key / query
    dtype (kv_cache.py:48-70, kernels/page_criticality.py:168);
  * threshold selection and tau clamping compare in fp32
    (kernels/selection_pack.py:150-198, kernels/tau_clamp.py:42-73).
Everything else (dot products, tau iterations, output sums) is evaluated in
float64, which is at least as accurate as the reference's fp32/fp16 Triton
arithmetic; tests compare to it with a stated tolerance.

Parity status of each function is recorded in its docstring ("pinned by"):
the CPU test-suite checks each one against closed forms, brute force,
library routines or invariants.
"""

from __future__ import annotations

import math
from statistics import NormalDist

import numpy as np

# ---------------------------------------------------------------------------
# dtype helpers
# ---------------------------------------------------------------------------

_DTYPES = ("fp32", "fp16", "bf16")


def round_to(x, dtype: str) -> np.ndarray:
    """Round float values to ``dtype`` (round-to-nearest-even), return float64.

    bf16 is emulated from fp32 bits (add 0x7FFF + lsb, truncate), which is the
    IEEE round-to-nearest-even conversion torch uses.
    """
    x = np.asarray(x, dtype=np.float64)
    if dtype == "fp32":
        return x.astype(np.float32).astype(np.float64)
    if dtype == "fp16":
        return x.astype(np.float16).astype(np.float64)
    if dtype == "bf16":
        f = x.astype(np.float32)
        u = f.view(np.uint32).astype(np.uint64)
        nan = np.isnan(f)
        lsb = (u >> 16) & 1
        u = ((u + 0x7FFF + lsb) >> 16) << 16
        out = u.astype(np.uint32).view(np.float32).astype(np.float64)
        return np.where(nan, np.nan, out)
    raise ValueError(f"unknown dtype {dtype!r}")


def f32(x) -> np.ndarray:
    return np.asarray(x, dtype=np.float64).astype(np.float32)


# ---------------------------------------------------------------------------
# a1 / a2: per-page key statistics
# ---------------------------------------------------------------------------

def page_stats(k: np.ndarray, page_size: int, dtype: str):
    """Per-page min/max/mean/std(population) of keys, clamped std >= 1e-6.

    Follows kv_cache.py:40-70 (initialize) and kv_cache.py:104-116 (the
    last-page recompute in append): for every page p the statistics are taken
    over rows [p*ps, min((p+1)*ps, S)).  Results are rounded to ``dtype``.

    k: [B, H, S, D] (values already representable in ``dtype``).
    Returns kmin, kmax, kmean, kstd, each [B, H, P, D] float64.
    Pinned by: brute-force numpy min/max/mean/std per page (tests).
    """
    B, H, S, D = k.shape
    P = (S + page_size - 1) // page_size
    pad = P * page_size - S
    kk = np.asarray(k, dtype=np.float64)
    if pad:
        kk = np.concatenate([kk, np.full((B, H, pad, D), np.nan)], axis=2)
    kk = kk.reshape(B, H, P, page_size, D)
    kmin = np.nanmin(kk, axis=3)
    kmax = np.nanmax(kk, axis=3)
    kmean = np.nanmean(kk, axis=3)
    kstd = np.sqrt(np.nanmean((kk - kmean[:, :, :, None, :]) ** 2, axis=3))
    kstd = np.maximum(kstd, 1e-6)
    return (round_to(kmin, dtype), round_to(kmax, dtype),
            round_to(kmean, dtype), round_to(kstd, dtype))


# ---------------------------------------------------------------------------
# a3: page criticality
# ---------------------------------------------------------------------------

def alibi_page_bonus(slopes: np.ndarray, num_pages: int, page_size: int,
                     seq_len: int, q_pos: int) -> np.ndarray:
    """fp32 ALiBi bonus per (head, page): slope * (min((p+1)ps-1, S-1) - q_pos).

    Follows kernels/page_criticality.py:157-166 (every op in fp32).
    """
    p = np.arange(num_pages, dtype=np.float32)
    last = np.minimum((p + np.float32(1)) * np.float32(page_size) - np.float32(1),
                      np.float32(seq_len - 1)).astype(np.float32)
    diff = (last - np.float32(q_pos)).astype(np.float32)
    return (f32(slopes)[:, None] * diff[None, :]).astype(np.float32)


def page_criticality(q: np.ndarray, kmin: np.ndarray, kmax: np.ndarray,
                     dtype: str, num_pages: int | None = None,
                     alibi_slopes=None, page_size: int = 16,
                     seq_len: int = 0, q_pos: int = 0) -> np.ndarray:
    """Upper-bound page score sum_d max(q_d*kmin_d, q_d*kmax_d) (+ ALiBi bonus).

    Follows kernels/page_criticality.py:61-104 with scale 1.0
    (apply_scaling=False at :111,148) and the output rounded to the query
    dtype (:168).  The bound chosen per element is kmax for q_d >= 0 and kmin
    otherwise (:88-95), which equals the max of the two products.

    q: [B, H, D]; kmin/kmax: [B, Hkv, P, D]; the first ``num_pages`` pages are
    scored (the in-progress last page is excluded by the caller passing P-1).
    The ALiBi slope of query head h is used for head h (the reference indexes
    its bonus table by kv head, identical under MHA, :100).
    Returns [B, H, num_pages] float64 rounded to ``dtype``.
    Pinned by: brute force max(q*kmin, q*kmax) sum (tests).
    """
    B, H, D = q.shape
    Hkv = kmin.shape[1]
    G = H // Hkv
    if num_pages is None:
        num_pages = kmin.shape[2]
    q64 = np.asarray(q, dtype=np.float64)
    kmn = np.repeat(np.asarray(kmin[:, :, :num_pages], np.float64), G, axis=1)
    kmx = np.repeat(np.asarray(kmax[:, :, :num_pages], np.float64), G, axis=1)
    bound = np.where(q64[:, :, None, :] >= 0, kmx, kmn)
    acc = np.einsum("bhpd,bhd->bhp", bound, q64)
    if alibi_slopes is not None:
        bonus = alibi_page_bonus(np.asarray(alibi_slopes), num_pages, page_size,
                                 seq_len, q_pos).astype(np.float64)
        # fp32 accumulator + fp32 bonus
        acc = f32(acc).astype(np.float64) + bonus[None, :, :]
        acc = f32(acc).astype(np.float64)
    return round_to(acc, dtype)


# ---------------------------------------------------------------------------
# a4: top-k page selection
# ---------------------------------------------------------------------------

def topk_pages(scores: np.ndarray, k: int) -> np.ndarray:
    """Indices of the ``k`` largest scores per row, returned in ascending order.

    Follows attention_topk.py:52-55 (torch.topk over the page axis).  torch
    leaves the order among equal scores unspecified; this build fixes it:
    among equal scores the lower page index wins.  NaN ranks above every
    number and -0.0 ranks below +0.0, as in torch.topk's radix select on the
    IEEE bit patterns.
    scores: [..., P]; returns int64 [..., k] sorted ascending.
    Pinned by: numpy lexsort brute force and torch.topk on tie-free rows.
    """
    s = np.asarray(scores, dtype=np.float64)
    lead = s.shape[:-1]
    P = s.shape[-1]
    flat = s.reshape(-1, P)
    out = np.empty((flat.shape[0], k), dtype=np.int64)
    idx = np.arange(P)
    for r in range(flat.shape[0]):
        row = flat[r]
        key = np.where(np.isnan(row), np.inf, row)
        nanflag = np.isnan(row).astype(np.int64)
        negzero = ((row == 0) & np.signbit(row)).astype(np.int64)
        # sort by (nan first, value desc, +0.0 before -0.0, index asc)
        order = np.lexsort((idx, negzero, -key, -nanflag))
        out[r] = np.sort(order[:k])
    return out.reshape(*lead, k)


def _page_order(row: np.ndarray) -> np.ndarray:
    """Pages of one score row from best to worst in topk_pages' order (NaN
    first, value descending, +0.0 before -0.0, lower index first)."""
    idx = np.arange(row.size)
    key = np.where(np.isnan(row), np.inf, row)
    nanflag = np.isnan(row).astype(np.int64)
    negzero = ((row == 0) & np.signbit(row)).astype(np.int64)
    return np.lexsort((idx, negzero, -key, -nanflag))


def topk_gqa_pages(scores: np.ndarray, num_kv_heads: int, k: int) -> np.ndarray:
    """Top-k pages of each KV head under GQA, ascending: [B, Hkv, k].

    The reference cannot run GQA top-k (attention_topk.py:52-71 packs per
    query head while kernels/adadecode_paged.py:600 requires kv-head keyed
    page tables).  This build's documented policy: a page's level is its best
    rank over the group's query heads (rank r = the r-th page of that head's
    topk_pages order), and the k pages of lowest level are taken, ties to the
    lower page index -- a round robin over the heads' own rankings.  It
    depends on each head's order only, so heads whose scores differ in scale
    or offset share the table fairly.  Reduces to topk_pages for MHA.
    Pinned by: topk_pages for G = 1, invariance to per-head positive affine
    maps, each head's top floor(k/G) kept, and a literal round-robin
    restatement on small inputs (tests).
    """
    s = np.asarray(scores, np.float64)
    B, H, P = s.shape
    G = H // num_kv_heads
    out = np.empty((B, num_kv_heads, k), dtype=np.int64)
    for b in range(B):
        for kvh in range(num_kv_heads):
            level = np.full(P, P, dtype=np.int64)
            for g in range(G):
                rank = np.empty(P, dtype=np.int64)
                rank[_page_order(s[b, kvh * G + g])] = np.arange(P)
                level = np.minimum(level, rank)
            out[b, kvh] = np.sort(np.lexsort((np.arange(P), level))[:k])
    return out


# ---------------------------------------------------------------------------
# a6: exact-mode paged entmax decode (histogram init + bracketed Halley)
# ---------------------------------------------------------------------------

BINS = 16


def decode_query_scale(alpha: float, head_dim: int, dtype: str) -> float:
    """(alpha-1)/sqrt(D) as the kernel's scalar operand (kernels/adadecode_paged.py:79,605).

    The constant is a Python float multiplied with a tensor of the input
    dtype; under Triton's scalar typing a Python scalar does not promote the
    tensor, so the product is taken in the input dtype: the constant itself is
    rounded to that dtype.
    """
    return float(round_to((alpha - 1.0) * (1.0 / math.sqrt(head_dim)), dtype))


def scaled_query(q: np.ndarray, alpha: float, dtype: str) -> np.ndarray:
    """q * (alpha-1)/sqrt(D) in the input dtype (kernels/adadecode_paged.py:97-98).

    For fp16/bf16 the product of two representable values is exact in fp32 and
    rounded once to the dtype; for fp32 it is the fp32 product.
    """
    D = q.shape[-1]
    c = decode_query_scale(alpha, D, dtype)
    prod = f32(q) * np.float32(c)
    return round_to(prod.astype(np.float64), dtype)


def compacted_rows(page_indices: np.ndarray, n: int, page_size: int) -> np.ndarray:
    """Cache rows of compacted tokens c in [0, n): page_indices[c//ps]*ps + c%ps.

    Follows kernels/adadecode_paged.py:20-31,116-119.
    """
    c = np.arange(n)
    return np.asarray(page_indices, np.int64)[c // page_size] * page_size + c % page_size


def head_scores(qs: np.ndarray, K: np.ndarray, rows: np.ndarray,
                alibi_slope: float = 0.0, alpha: float = 1.5,
                q_idx: int = 0) -> np.ndarray:
    """Entmax-scaled scores s_c = qs . K[row_c] (+ (alpha-1)*slope*(row_c - q_idx)).

    Follows kernels/adadecode_paged.py:121-127 (float64 dot product).
    """
    s = np.asarray(K, np.float64)[rows] @ np.asarray(qs, np.float64)
    if alibi_slope != 0.0:
        slope = float(np.float32(np.float32(alibi_slope) * np.float32(alpha - 1.0)))
        s = s + slope * (rows.astype(np.float64) - q_idx)
    return s


def histogram_init(s: np.ndarray, alpha: float):
    """Global max, 16-bin histogram and tau bracket init for one head.

    Follows kernels/adadecode_paged.py:210-243 (binning with truncation toward
    zero, so values in (t0-1/16, t0) land in bin 0), kernels/adadecode.py:218-232
    (max reduce, -1e6 floor), :351-371 (hist reduce), :381-426 (init) with
    init_tau_alpha2_tinit (:38-51), init_tau_alpha15_tinit (:54-71) and
    init_tau_generic_find_bin (:74-112).
    Returns (t, t_lo, t_hi, gmax, hist).
    Pinned by: for scores on the bins' lower edges (and a unique maximum) the
    alpha=2 and alpha=1.5 init equals the exact root (brentq); the truncation
    quirk case; convergence of the iteration to exact entmax.
    """
    gmax = max(-1.0e6, float(np.max(s))) if s.size else -1.0e6
    t0 = gmax - 1.0
    hist = np.zeros(BINS, dtype=np.int64)
    if s.size:
        proj = (s - t0) * BINS
        b = np.trunc(proj)
        b = np.minimum(b, BINS - 1)
        ok = b >= 0
        np.add.at(hist, b[ok].astype(np.int64), 1)
    if alpha == 2.0 or alpha == 1.5:
        sum_z, sum_k, sum_z2 = 1.0, 1.0, 1.0
        for sj in range(BINS - 1, -1, -1):
            c_bin = float(hist[sj]) - (1.0 if sj == BINS - 1 else 0.0)
            c_tau = sj / BINS
            new_z = sum_z + c_bin * c_tau
            new_k = sum_k + c_bin
            if alpha == 2.0:
                if (new_z - new_k * c_tau) < 1.0:
                    sum_z, sum_k = new_z, new_k
            else:
                new_z2 = sum_z2 + c_bin * (c_tau * c_tau)
                if new_k * c_tau * c_tau - 2.0 * new_z * c_tau + new_z2 < 1.0:
                    sum_z, sum_k, sum_z2 = new_z, new_k, new_z2
        if alpha == 2.0:
            t_init = gmax + (sum_z - 1.0) / sum_k - 1.0
        else:
            disc = sum_z * sum_z - sum_k * (sum_z2 - 1.0)
            t_init = gmax + (sum_z - math.sqrt(disc) if disc >= 0 else math.nan) / sum_k - 1.0
        t_lo = t_init
        t_hi = t_init + 1.0 / BINS
    else:
        counts = hist.astype(np.float64)
        counts[BINS - 1] -= 1.0
        p = 1.0 / (alpha - 1.0)
        lo, hi, found, b_idx = 0, BINS - 1, 0, 0
        bins = np.arange(BINS)
        for _ in range(5):
            mid = int((lo + hi) * 0.5)
            off = bins - mid
            mask = off >= 0
            zL = off / BINS
            zU = (off + 1.0) / BINS
            termL = np.where(mask & (zL > 0), np.where(zL > 0, zL, 1.0) ** p, 0.0)
            termU = np.where(mask, zU ** p, 0.0)
            fL = float(np.sum(counts * termL)) - 1.0
            fU = float(np.sum(counts * termU)) - 1.0
            go_right = fL > 0.0
            go_left = fU < 0.0
            bracket = (not go_right) and (not go_left)
            if found == 0:
                if bracket:
                    b_idx, found = mid, 1
                if go_right:
                    lo = mid + 1
                if go_left:
                    hi = mid - 1
        b_sel = b_idx if found == 1 else min(lo, BINS - 1)
        t_lo = t0 + b_sel / BINS
        t_hi = t0 + min(b_sel + 1, BINS) / BINS
    t = 0.5 * (t_lo + t_hi)
    return t, t_lo, t_hi, gmax, hist


def entmax_accumulators(s: np.ndarray, t: float, alpha: float):
    """(acc0, acc1, acc2) of kernels/adadecode_paged.py:357-372 at threshold t.

    Pinned by: f = acc0 - 1, f' = -acc1/(alpha-1) and f'' through the Halley
    step checks (finite differences of the brute-force f).
    """
    act = s - t
    m = act > 0
    a = act[m]
    if alpha == 2.0:
        return float(np.sum(a)), float(np.count_nonzero(m)), 0.0
    if alpha == 1.5:
        return float(np.sum(a * a)), float(np.sum(a)), float(np.count_nonzero(m))
    c0 = 1.0 / (alpha - 1.0)
    return (float(np.sum(a ** c0)), float(np.sum(a ** (c0 - 1.0))),
            float(np.sum(a ** (c0 - 2.0))))


def halley_bisect_update(t, t_lo, t_hi, acc0, acc1, acc2, alpha):
    """Bracketed Halley step, kernels/adadecode.py:12-35 (EPS 1e-6).

    Pinned by: one step equals t - 2ff'/(2f'^2 - ff'') with f, f', f'' from
    finite differences of the brute-force f; bracket update by sign(f); the
    midpoint fallback; at alpha=2 one step lands on the sparsemax root.
    """
    c0 = 1.0 / (alpha - 1.0)
    c1 = c0 - 1.0
    ff = acc0 - 1.0
    df = -c0 * acc1
    ddf = c0 * c1 * acc2
    if ff > 0:
        t_lo = t
    if ff < 0:
        t_hi = t
    den = 2 * df * df - ff * ddf
    with np.errstate(all="ignore"):
        new_t = t - (2 * ff * df) / den if den != 0 else (
            math.nan if (2 * ff * df) == 0 else math.copysign(math.inf, -(2 * ff * df)))
    good = (new_t > t_lo - 1e-6) and (new_t < t_hi + 1e-6)
    t = new_t if good else 0.5 * (t_lo + t_hi)
    return t, t_lo, t_hi


def entmax_weights(s: np.ndarray, t: float, alpha: float) -> np.ndarray:
    """p_c = [s_c - t]_+^(1/(alpha-1)) (kernels/adadecode_paged.py:487-504)."""
    act = s - t
    m = act > 0
    p = np.zeros_like(s)
    if alpha == 2.0:
        p[m] = act[m]
    elif alpha == 1.5:
        p[m] = act[m] * act[m]
    else:
        p[m] = act[m] ** (1.0 / (alpha - 1.0))
    return p


def solve_tau_exact_iterative(s: np.ndarray, alpha: float, niter: int):
    """tau after histogram init + ``niter`` bracketed Halley steps (a6 stages 1-5).

    Follows kernels/adadecode_paged.py:650-732.
    """
    t, t_lo, t_hi, _, _ = histogram_init(s, alpha)
    for _ in range(niter):
        a0, a1, a2 = entmax_accumulators(s, t, alpha)
        t, t_lo, t_hi = halley_bisect_update(t, t_lo, t_hi, a0, a1, a2, alpha)
    return t


def paged_entmax_decode(q, K, V, page_indices, cache_seqlens, page_size, alpha,
                        niter, dtype, alibi_slopes=None, q_seqlens=None,
                        tau_given=None, tau_iters=0):
    """Paged split-KV entmax decode for every (b, h), float64.

    Exact mode (``tau_given is None``) follows kernels/adadecode_paged.py:567-762:
    scores over the compacted token list, histogram init, ``niter`` bracketed
    Halley steps, out = sum_c [s_c - tau]_+^(1/(alpha-1)) v_c (not renormalised).
    Given-tau mode follows kernels/adadecode_paged_gaussian_tau.py:192-331:
    ``tau_iters`` unbounded Halley/Newton steps from ``tau_given`` (:12-53) then
    the same weighted sum.

    q: [B, H, D]; K, V: [B, Hkv, S, D]; page_indices: [B, Hkv, n_slots] int;
    cache_seqlens: [B, Hkv] compacted token counts; q_seqlens: [B] (ALiBi only).
    Returns (out [B, H, D] float64, tau [B, H] float64).
    Pinned by: exact sort-based entmax over the same tokens once converged,
    and brute-force restatement checks (tests).
    """
    B, H, D = q.shape
    Hkv = K.shape[1]
    G = H // Hkv
    qs = scaled_query(q, alpha, dtype)
    out = np.zeros((B, H, D))
    taus = np.zeros((B, H))
    for b in range(B):
        for h in range(H):
            kvh = h // G
            n = int(cache_seqlens[b, kvh])
            rows = compacted_rows(page_indices[b, kvh], n, page_size)
            slope = 0.0 if alibi_slopes is None else float(alibi_slopes[h])
            q_idx = (int(q_seqlens[b]) - 1) if q_seqlens is not None else 0
            s = head_scores(qs[b, h], K[b, kvh], rows, slope, alpha, q_idx)
            if tau_given is None:
                t = solve_tau_exact_iterative(s, alpha, niter)
            else:
                t = float(tau_given[b, h])
                for _ in range(tau_iters):
                    a0, a1, a2 = entmax_accumulators(s, t, alpha)
                    t = halley_unbounded_update(t, a0, a1, a2, alpha)
            p = entmax_weights(s, t, alpha)
            out[b, h] = p @ np.asarray(V[b, kvh], np.float64)[rows] if n else 0.0
            taus[b, h] = t
    return out, taus


def halley_unbounded_update(t, acc0, acc1, acc2, alpha):
    """kernels/adadecode_paged_gaussian_tau.py:12-53 (Halley, else Newton, else keep).

    Pinned by: one step equals textbook Halley on the brute-force f (finite
    differences), alpha=1.5; lands exactly on the sparsemax root at alpha=2;
    cubic error contraction near the root.
    """
    c0 = 1.0 / (alpha - 1.0)
    c1 = c0 - 1.0
    ff = acc0 - 1.0
    df = -c0 * acc1
    ddf = c0 * c1 * acc2
    hden = 2.0 * df * df - ff * ddf
    if abs(hden) > 1e-12:
        tn = t - (2.0 * ff * df) / hden
    elif abs(df) > 1e-12:
        tn = t - ff / df
    else:
        tn = t
    if not (tn == tn and abs(tn) < 1e20):
        tn = t
    return tn


# ---------------------------------------------------------------------------
# exact entmax (sort based) — the mathematical pin for a6
# ---------------------------------------------------------------------------

def entmax_tau_exact(s: np.ndarray, alpha: float) -> float:
    """Exact threshold tau with sum_c [s_c - tau]_+^(1/(alpha-1)) = 1.

    alpha=2: sparsemax, Martins & Astudillo (2016): sort descending, the
    support size k is the largest k with 1 + k*s_(k) > sum_{i<=k} s_(i), and
    tau = (sum_{i<=k} s_(i) - 1)/k.
    alpha=1.5: Peters, Niculae & Martins (2019), sort-based entmax-1.5: for the
    sorted prefix of size k, tau_k = mean_k - sqrt((1 - k*(meansq_k - mean_k^2))/k);
    the support is the largest k with tau_k <= s_(k).
    other alpha: bisection on [max-1, max] to float64 resolution.
    ``s`` is already in the (alpha-1)-scaled space.
    """
    s = np.sort(np.asarray(s, np.float64))[::-1]
    n = s.size
    if n == 0:
        return math.nan
    k = np.arange(1, n + 1)
    if alpha == 2.0:
        cs = np.cumsum(s)
        supp = 1.0 + k * s > cs
        kk = int(np.nonzero(supp)[0][-1]) + 1
        return (cs[kk - 1] - 1.0) / kk
    if alpha == 1.5:
        mean = np.cumsum(s) / k
        meansq = np.cumsum(s * s) / k
        ss = k * (meansq - mean * mean)
        delta = (1.0 - ss) / k
        tau = mean - np.sqrt(np.clip(delta, 0.0, None))
        supp = tau <= s
        kk = int(np.nonzero(supp)[0][-1]) + 1
        return float(tau[kk - 1])
    lo, hi = s[0] - 1.0, s[0]
    e = 1.0 / (alpha - 1.0)
    for _ in range(200):
        mid = 0.5 * (lo + hi)
        f = np.sum(np.clip(s - mid, 0.0, None) ** e) - 1.0
        if f > 0:
            lo = mid
        else:
            hi = mid
    return 0.5 * (lo + hi)


def entmax_exact(s: np.ndarray, alpha: float) -> np.ndarray:
    """Exact entmax probabilities over scores already scaled by (alpha-1)."""
    t = entmax_tau_exact(s, alpha)
    return entmax_weights(np.asarray(s, np.float64), t, alpha)


def entmax_rows(x: np.ndarray, alpha: float) -> np.ndarray:
    """Row-wise alpha-entmax over the last axis of x (unscaled inputs).

    kernels/triton_entmax.py:364-533 scales x by (alpha-1) (:401-409, :472)
    and writes [z - tau]_+^(1/(alpha-1)) (:514-533) after ``n_iter`` hybrid
    steps; this restatement uses the exact tau (entmax_exact), the limit the
    reference's iterations approach.  Pinned by: entmax_tau_exact's checks.
    """
    x = np.asarray(x, np.float64)
    flat = x.reshape(-1, x.shape[-1])
    out = np.stack([entmax_exact((alpha - 1.0) * r, alpha) for r in flat])
    return out.reshape(x.shape)


def entmax_rows_backward(y: np.ndarray, dy: np.ndarray, alpha: float) -> np.ndarray:
    """Vector-Jacobian product of row-wise entmax at output y.

    kernels/triton_entmax.py:536-612: u = y^(2-alpha) on {y > 0},
    dx = u * dy - (sum u dy / sum u) * u.  Pinned by: central finite
    differences of entmax_rows (tests).
    """
    y = np.asarray(y, np.float64)
    dy = np.asarray(dy, np.float64)
    u = np.where(y > 0, np.abs(y) ** (2.0 - alpha), 0.0)
    scalar = (u * dy).sum(-1, keepdims=True) / u.sum(-1, keepdims=True)
    return u * dy - scalar * u


def dense_entmax_decode(q, K, V, cache_seqlens, alpha, niter, dtype, alibi_slopes=None,
                        token_positions=None, q_seqlens=None):
    """Dense (non-paged) decode of kernels/adadecode.py:754-1016, float64.

    Head (b, h) attends to rows [0, cache_seqlens[b]) of K[b, h // G]; scores
    use the dtype-rounded scaled query (:161-163); ALiBi adds
    (alpha-1) * slope_h * (token_positions[b, kvh, j] - q_idx) with
    q_idx = q_seqlens[b] - 1, q_seqlens defaulting to cache_seqlens (:188-205,
    :787-791); tau from the 16-bin histogram init and ``niter`` bracketed
    Halley steps (:382-592); out = sum_j [s_j - tau]_+^(1/(alpha-1)) v_j.
    q: [B, H, D]; K, V: [B, Hkv, S, D].  Returns (out [B, H, D], tau [B, H]).
    Pinned by: paged_entmax_decode with an identity page table (same tokens,
    same tau trajectory) and entmax_exact once converged (tests).
    """
    B, H, D = q.shape
    Hkv = K.shape[1]
    G = H // Hkv
    qs = scaled_query(q, alpha, dtype)
    out = np.zeros((B, H, D))
    taus = np.zeros((B, H))
    for b in range(B):
        n = int(cache_seqlens[b])
        q_idx = int(q_seqlens[b] if q_seqlens is not None else cache_seqlens[b]) - 1
        for h in range(H):
            kvh = h // G
            rows = np.arange(n)
            s = np.asarray(K[b, kvh], np.float64)[rows] @ np.asarray(qs[b, h], np.float64)
            if alibi_slopes is not None:
                slope = float(np.float32(np.float32(alibi_slopes[h]) * np.float32(alpha - 1.0)))
                pos = rows if token_positions is None else np.asarray(token_positions[b, kvh])[rows]
                s = s + slope * (pos.astype(np.float64) - q_idx)
            t = solve_tau_exact_iterative(s, alpha, niter)
            p = entmax_weights(s, t, alpha)
            out[b, h] = p @ np.asarray(V[b, kvh], np.float64)[rows] if n else 0.0
            taus[b, h] = t
    return out, taus


# ---------------------------------------------------------------------------
# a7: Gaussian page statistics
# ---------------------------------------------------------------------------

def gaussian_page_stats(q, kmean, kstd, pages_for_stats):
    """Per-page score mean/variance and per-head global moments.

    Follows kernels/gaussian_page_stats.py:8-121:
      mu_p  = sum_d (q_d*scale) * kmean_pd,   scale = 1/sqrt(D) in fp32
      var_p = sum_d (q_d*scale)^2 * kstd_pd^2
      mu_g = mean_p mu_p, mean_var = mean_p var_p,
      var_means = max(mean_p mu_p^2 - mu_g^2, 0)
    and gaussian_utils.py:155-161 (nan_to_num, sigma_g clamp >= 1e-6).
    q: [B, H, D]; kmean/kstd: [B, Hkv, P, D] (Hkv == H in the reference,
    kernels/gaussian_page_stats.py:148-149; this build maps q head h to kv
    head h // (H/Hkv)).
    Returns dict with mu_p, sigma_p ([B,H,P'] float64), mu_g, sigma_g,
    mean_var, var_means ([B,H]).
    Pinned by: numpy var/mean identities and a brute-force loop (tests).
    """
    B, H, D = q.shape
    Hkv = kmean.shape[1]
    G = H // Hkv
    scale = np.float32(1.0 / math.sqrt(D))
    qsc = (f32(q) * scale).astype(np.float64)
    km = np.repeat(np.asarray(kmean[:, :, :pages_for_stats], np.float64), G, axis=1)
    ks = np.repeat(np.asarray(kstd[:, :, :pages_for_stats], np.float64), G, axis=1)
    mu_p = np.einsum("bhpd,bhd->bhp", km, qsc)
    var_p = np.einsum("bhpd,bhd->bhp", ks * ks, qsc * qsc)
    mu_g = mu_p.mean(axis=-1)
    mean_var = var_p.mean(axis=-1)
    var_means = np.maximum((mu_p * mu_p).mean(axis=-1) - mu_g * mu_g, 0.0)
    mu_g = np.nan_to_num(mu_g, nan=0.0, posinf=0.0, neginf=0.0)
    sigma_g = np.nan_to_num(np.sqrt(mean_var + var_means), nan=1e-6, posinf=1e6,
                            neginf=1e-6)
    sigma_g = np.maximum(sigma_g, 1e-6)
    return {"mu_p": mu_p, "sigma_p": np.sqrt(var_p), "var_p": var_p, "mu_g": mu_g,
            "sigma_g": sigma_g, "mean_var": mean_var, "var_means": var_means}


def auto_selection_margins(sigma_g: np.ndarray):
    """(safety_margin_z, max_quantile) from gaussian_utils.py:163-169.

    sigma_bar = mean over all (b, h) of sigma_g; low = sigma_bar < 1.5;
    safety_margin_z = (0.01 if low else 0.05) * sigma_bar;
    max_quantile = 0.99 if low else 0.995.
    """
    sbar = float(np.mean(sigma_g))
    low = sbar < 1.5
    return (0.01 if low else 0.05) * sbar, (0.99 if low else 0.995)


def page_quantile_z(quantile: float, page_size: int) -> float:
    """Normal quantile of quantile**(1/ps) (kernels/selection_pack.py:238-239)."""
    return NormalDist().inv_cdf(quantile ** (1.0 / page_size))


# ---------------------------------------------------------------------------
# a8: single-Gaussian tau solver
# ---------------------------------------------------------------------------

def _phi(x):
    return math.exp(-0.5 * x * x) / math.sqrt(2.0 * math.pi)


def _Phi(x):
    return 0.5 * (1.0 + math.erf(x / math.sqrt(2.0)))


def gaussian_constraint(tau, mu_g, sigma_g, n, alpha):
    """f(tau) = n*E[[(alpha-1)S - tau]_+^(1/(alpha-1))] - 1 and derivatives.

    Closed forms of kernels/tau_solver_gpu.py:20-77 (sigma_y >= 1e-10):
    alpha=2: E = mu_y*Phi(t) + sigma_y*phi(t), f' = -n*Phi, f'' = n*phi/sigma_y;
    alpha=1.5: E = (mu_y^2+sigma_y^2)*Phi(t) + mu_y*sigma_y*phi(t),
    f' = -2n*m1, f'' = 2n*Phi; mu_y = (alpha-1)*mu_g - tau, sigma_y = (alpha-1)*sigma_g.
    Pinned by: numerical integration of the truncated moments (tests).
    """
    a = alpha - 1.0
    sy = max(a * sigma_g, 1e-10)
    my = a * mu_g - tau
    t = my / sy
    ph, Ph = _phi(t), _Phi(t)
    m0 = Ph
    m1 = my * Ph + sy * ph
    m2 = (my * my + sy * sy) * Ph + my * sy * ph
    if alpha == 2.0:
        return n * m1 - 1.0, -n * m0, n * ph / sy
    if alpha == 1.5:
        return n * m2 - 1.0, -2.0 * n * m1, 2.0 * n * m0
    m3 = (my ** 3 + 3.0 * my * sy * sy) * Ph + (sy ** 3 + 2.0 * my * my * sy) * ph
    return n * m3 - 1.0, -3.0 * n * m2, 6.0 * n * m1


def tau_single_gaussian(mu_g, sigma_g, n, alpha, iterations=120, tol=1e-6):
    """Bracketed Halley root of f(tau) per head, float64.

    Follows kernels/tau_solver_gpu.py:79-125 (bracket (alpha-1)mu_g +-
    (alpha-1)sigma_g(sqrt(2 ln(n+1)) + 8), ``iterations`` fixed steps, Halley
    when |2f'^2 - f f''| > 1e-18 else Newton with f' <= -1e-12, candidates
    outside (lo, hi) or non-finite replaced by the midpoint, tau = candidate
    when |f(candidate)| <= tol else the new midpoint).
    mu_g, sigma_g: arrays of any shape; returns the same shape.
    """
    mu = np.asarray(mu_g, np.float64)
    sg = np.asarray(sigma_g, np.float64)
    out = np.empty_like(mu)
    lnf = math.sqrt(2.0 * math.log(n + 1.0))
    a = alpha - 1.0
    for i in np.ndindex(mu.shape):
        m, s = float(mu[i]), max(float(sg[i]), 1e-6)
        r = a * s * (lnf + 8.0)
        lo, hi = a * m - r, a * m + r
        t = 0.5 * (lo + hi)
        for _ in range(iterations):
            f, fp, fpp = gaussian_constraint(t, m, s, n, alpha)
            mid = 0.5 * (lo + hi)
            den = 2.0 * fp * fp - f * fpp
            if abs(den) > 1e-18:
                step = 2.0 * f * fp / den
            else:
                step = f / min(fp, -1e-12)
            cand = t - step
            if not (cand == cand and abs(cand) < 1e20 and lo < cand < hi):
                cand = mid
            fc = gaussian_constraint(cand, m, s, n, alpha)[0]
            if fc > 0.0:
                lo = cand
            else:
                hi = cand
            t = cand if abs(fc) <= tol else 0.5 * (lo + hi)
        out[i] = t
    return out


# ---------------------------------------------------------------------------
# a9: page-mixture tau solver (ALiBi)
# ---------------------------------------------------------------------------

def alibi_page_mean_bias(slopes, pages_for_stats, seq_len, page_size):
    """slope_h * (min(p*ps + (ps-1)/2, seq_len_for_stats... ) - q_pos).

    Follows gaussian_utils.py:142-153: page_mean_pos = p*ps + (ps-1)/2 clamped
    to seq_len_for_stats - 1, q_pos = seq_len - 1.  Returns [H, P'] float64.
    """
    slen_stats = pages_for_stats * page_size
    pos = np.minimum(np.arange(pages_for_stats) * page_size + (page_size - 1) / 2.0,
                     slen_stats - 1)
    return np.asarray(slopes, np.float64)[:, None] * (pos[None, :] - (seq_len - 1))


def _mixture_f(tau, mu, sg, cnt, alpha):
    a = alpha - 1.0
    sy = np.maximum(a * sg, 1e-10)
    my = a * mu - tau
    t = my / sy
    ph = np.exp(-0.5 * t * t) / math.sqrt(2 * math.pi)
    from scipy.special import erf
    Ph = 0.5 * (1.0 + erf(t / math.sqrt(2.0)))
    m0 = Ph
    m1 = my * Ph + sy * ph
    m2 = (my * my + sy * sy) * Ph + my * sy * ph
    if alpha == 2.0:
        e, d1, d2 = m1, -m0, ph / sy
    elif alpha == 1.5:
        e, d1, d2 = m2, -2.0 * m1, 2.0 * m0
    else:
        m3 = (my ** 3 + 3.0 * my * sy * sy) * Ph + (sy ** 3 + 2.0 * my * my * sy) * ph
        e, d1, d2 = m3, -3.0 * m2, 6.0 * m1
    return (float(np.sum(cnt * e)) - 1.0, float(np.sum(cnt * d1)),
            float(np.sum(cnt * d2)))


def tau_page_mixture(mu_p, sigma_p, count, alpha, max_iter=40, tol=1e-6):
    """Root of sum_p c_p E_p[[(alpha-1)S_p - tau]_+^(1/(alpha-1))] = 1 per row.

    Follows kernels/tau_mixture_solver_triton.py:81-165 (uniform page count):
    bracket max_y +- max_sigma_y(sqrt(2 ln(N+1)) + 8), 8 bracket expansions
    with doubling radius, then ``max_iter`` bracketed Halley steps.
    mu_p, sigma_p: [..., P]; returns [...] float64.
    Pinned by: at P=1 it reduces to the single-Gaussian solver with n=count.
    """
    mu = np.asarray(mu_p, np.float64)
    sg = np.maximum(np.asarray(sigma_p, np.float64), 1e-6)
    lead = mu.shape[:-1]
    P = mu.shape[-1]
    out = np.zeros(lead)
    a = alpha - 1.0
    for i in np.ndindex(lead):
        m, s = mu[i], sg[i]
        cnt = np.full(P, float(count))
        total = max(cnt.sum(), 1.0)
        lnf = math.sqrt(2.0 * math.log(total + 1.0))
        max_y = float(np.max(a * m))
        max_s = max(float(np.max(a * s)), 1e-6)
        r = max_s * (lnf + 8.0)
        lo, hi = max_y - r, max_y + r
        for _ in range(8):
            flo = _mixture_f(lo, m, s, cnt, alpha)[0]
            fhi = _mixture_f(hi, m, s, cnt, alpha)[0]
            if flo <= 0.0:
                lo -= r
            if fhi > 0.0:
                hi += r
            r *= 2.0
        t = 0.5 * (lo + hi)
        for _ in range(max_iter):
            f, fp, fpp = _mixture_f(t, m, s, cnt, alpha)
            mid = 0.5 * (lo + hi)
            den = 2.0 * fp * fp - f * fpp
            if abs(den) > 1e-18:
                step = 2.0 * f * fp / den
            else:
                step = f / min(fp, -1e-12)
            cand = t - step
            if not (cand == cand and abs(cand) < 1e20 and lo < cand < hi):
                cand = mid
            fc = _mixture_f(cand, m, s, cnt, alpha)[0]
            if fc > 0.0:
                lo = cand
            else:
                hi = cand
            t = cand if abs(fc) <= tol else 0.5 * (lo + hi)
        out[i] = t
    return out


# ---------------------------------------------------------------------------
# a10 / a11 / a12: threshold selection, tau clamp, compacted lengths
# ---------------------------------------------------------------------------

def _fma32(a, b, c):
    """fp32 fused multiply-add emulated in float64 (exact product, one rounding)."""
    return f32(np.asarray(a, np.float64) * np.asarray(b, np.float64)
               + np.asarray(c, np.float64))


def tau_floor_fp32(mu_p, sigma_p, tau_hat, sigma_g, alpha, safety_margin_z,
                   frac, pages_for_stats):
    """tau_floor of kernels/selection_pack.py:150-159 in fp32 (per row).

    upper = mean_p(mu_p + 1.5 sigma_p); thr = tau_hat/(alpha-1);
    delta = max(smz*sigma_g, frac*max(thr - upper, 0)); tau_floor = tau_hat - delta*(alpha-1).
    The page sum is taken in float64 (the reference's fp32 reduction order is
    not specified); callers compare tau_floor with a tolerance.
    """
    am1 = np.float32(alpha - 1.0)
    mu = np.asarray(mu_p, np.float64)[..., :pages_for_stats]
    sg = np.asarray(sigma_p, np.float64)[..., :pages_for_stats]
    upper = f32(np.sum(f32(mu + 1.5 * sg).astype(np.float64), axis=-1) / pages_for_stats)
    thr = f32(tau_hat) / am1
    sig_delta = np.float32(safety_margin_z) * f32(sigma_g)
    excess = np.maximum(f32(thr - upper), np.float32(0))
    tau_delta = np.float32(frac) * excess
    delta = np.maximum(sig_delta, tau_delta).astype(np.float32)
    return f32(f32(tau_hat).astype(np.float64) - delta.astype(np.float64) * float(am1))


def select_gaussian_pages(mu_p, sigma_p, tau_floor, alpha, z_page,
                          pages_for_stats, num_pages):
    """Threshold mask + ascending pack + last-page sentinel, fp32 compares.

    Follows kernels/selection_pack.py:160-198: page p < P' is selected iff
    fl32((alpha-1) * fma32(z_page, sigma_p, mu_p)) > tau_floor; the selected
    pages are packed in ascending order; when num_pages > P' the last page
    (num_pages-1) is appended.  Bit-exact given identical fp32 inputs.
    Returns (indices list per row as int64 arrays, counts [...]).
    """
    am1 = np.float32(alpha - 1.0)
    mu = f32(np.asarray(mu_p)[..., :pages_for_stats])
    sg = f32(np.asarray(sigma_p)[..., :pages_for_stats])
    sbar = _fma32(np.float32(z_page), sg, mu)
    score = (am1 * sbar).astype(np.float32)
    sel = score > f32(tau_floor)[..., None]
    lead = sel.shape[:-1]
    counts = np.zeros(lead, dtype=np.int64)
    packed = np.empty(lead, dtype=object)
    for i in np.ndindex(lead):
        idx = np.nonzero(sel[i])[0]
        if num_pages > pages_for_stats:
            idx = np.concatenate([idx, [num_pages - 1]])
        packed[i] = idx.astype(np.int64)
        counts[i] = idx.size
    return packed, counts


def tau_clamp(tau, mu_p, sigma_p, packed, counts, tau_floor, alpha, z_clamp,
              pages_for_stats, eps=1e-4):
    """Clamp tau to the selected pages' score caps, fp32.

    Follows kernels/tau_clamp.py:42-73: cap_p = mu_p + (z_clamp*sigma_p)*(1/3)
    (the last multiply-add fused); upper = max(fma(alpha-1, max_{selected
    p < P'} cap_p, -eps), tau_floor);
    tau <- min(tau, upper) when any valid page is selected.
    """
    am1 = np.float32(alpha - 1.0)
    third = np.float32(0.3333333333333333)
    out = f32(tau).copy()
    for i in np.ndindex(out.shape):
        idx = np.asarray(packed[i][: counts[i]], np.int64)
        idx = idx[(idx >= 0) & (idx < pages_for_stats)]
        if idx.size == 0:
            continue
        mu = f32(np.asarray(mu_p)[i][idx])
        sg = f32(np.asarray(sigma_p)[i][idx])
        zs = (np.float32(z_clamp) * sg).astype(np.float32)
        cap = _fma32(zs, third, mu)
        cmax = np.float32(np.max(cap))
        upper = np.float32(_fma32(am1, cmax, -np.float32(eps)))
        if tau_floor is not None:
            upper = max(upper, np.float32(f32(tau_floor)[i]))
        out[i] = min(out[i], upper)
    return out.astype(np.float64)


def cache_seqlens_from_counts(counts, page_size, last_page_size):
    """max(count-1, 0)*ps + last_page_size (kernels/selection_pack.py:7-20)."""
    c = np.asarray(counts, np.int64)
    return np.maximum(c - 1, 0) * page_size + last_page_size


def last_page_size(seq_len, page_size):
    """attention_gaussian.py:99."""
    if seq_len > page_size:
        return seq_len - (math.ceil(seq_len / page_size) - 1) * page_size
    return seq_len


# ---------------------------------------------------------------------------
# end-to-end steps (used by the CPU baseline and end-to-end tests)
# ---------------------------------------------------------------------------

def topk_decode_step(q, K, V, stats, token_budget, page_size, alpha, niter,
                     dtype, alibi_slopes=None):
    """One top-k decode step over an already-appended cache (attention_topk.py:8-100).

    q: [B,H,D]; K,V: [B,Hkv,S,D]; stats = (kmin, kmax, ...).
    Returns (out [B,H,D], page_indices [B,Hkv,k+1], scores [B,H,P']).
    """
    B, H, D = q.shape
    Hkv, S = K.shape[1], K.shape[2]
    P = (S + page_size - 1) // page_size
    k = min(token_budget // page_size, P - 1)
    kmin, kmax = stats[0], stats[1]
    scores = page_criticality(q, kmin, kmax, dtype, num_pages=P - 1,
                              alibi_slopes=alibi_slopes, page_size=page_size,
                              seq_len=S, q_pos=S - 1)
    sel = topk_gqa_pages(scores, Hkv, k)
    pidx = np.concatenate([sel, np.full((B, Hkv, 1), P - 1)], axis=2)
    lps = S - (P - 1) * page_size
    seqlens = np.full((B, Hkv), k * page_size + lps)
    qsl = np.full((B,), S)
    out, _ = paged_entmax_decode(q, K, V, pidx, seqlens, page_size, alpha, niter,
                                 dtype, alibi_slopes=alibi_slopes, q_seqlens=qsl)
    return out, pidx, scores


def gaussian_decode_step(q, K, V, kmean, kstd, page_size, alpha, dtype,
                         tau_mode="corrected", niter=2, tau_iters=None,
                         clamp=True, frac=0.2, clamp_quantile=0.5):
    """One Gaussian-aware decode step (attention_gaussian.py:20-144), no ALiBi.

    Returns dict with out, packed indices, counts, tau values and stats.
    """
    B, H, D = q.shape
    S = K.shape[2]
    P = kmean.shape[2]
    pfs = P - 1 if P > 1 else P
    last_tok = S - (P - 1) * page_size if P > 1 else 0
    n_stats = S - last_tok
    st = gaussian_page_stats(q, kmean, kstd, pfs)
    smz, mq = auto_selection_margins(st["sigma_g"])
    tau_hat = tau_single_gaussian(st["mu_g"], st["sigma_g"], n_stats, alpha)
    tfloor = tau_floor_fp32(st["mu_p"], st["sigma_p"], tau_hat, st["sigma_g"],
                            alpha, smz, frac, pfs)
    z_page = page_quantile_z(mq, page_size)
    packed, counts = select_gaussian_pages(st["mu_p"], st["sigma_p"], tfloor, alpha,
                                           z_page, pfs, P)
    tau = tau_hat
    if tau_mode != "exact" and clamp:
        z_c = page_quantile_z(clamp_quantile, page_size)
        tau = tau_clamp(tau_hat, st["mu_p"], st["sigma_p"], packed, counts, tfloor,
                        alpha, z_c, pfs)
    lps = last_page_size(S, page_size)
    seqlens = cache_seqlens_from_counts(counts, page_size, lps)
    maxc = int(counts.max()) if counts.size else 0
    pidx = np.zeros((B, H, max(maxc, 1)), dtype=np.int64)
    for i in np.ndindex(counts.shape):
        pidx[i][: counts[i]] = packed[i]
    if tau_mode == "exact":
        out, taus = paged_entmax_decode(q, K, V, pidx, seqlens, page_size, alpha,
                                        niter, dtype)
    else:
        if tau_iters is None:
            tau_iters = 0 if tau_mode == "fixed" else 1
        out, taus = paged_entmax_decode(q, K, V, pidx, seqlens, page_size, alpha,
                                        0, dtype, tau_given=tau, tau_iters=tau_iters)
    return {"out": out, "packed": packed, "counts": counts, "tau_hat": tau_hat,
            "tau_floor": tfloor, "tau": tau, "tau_final": taus, "stats": st,
            "seqlens": seqlens, "smz": smz, "max_quantile": mq}
