"""Launchers for the HIP kernels, one per reference kernel module.

Each launcher validates shapes and dtypes on the host (raising the same
exception types the reference raises: AssertionError for shape asserts,
ValueError for bad parameters), then calls one entry point of the C ABI on
the current HIP stream.  No launcher synchronises with the device.
"""

from __future__ import annotations

import math
from statistics import NormalDist

from typing import NamedTuple

import torch

from ._lib import call, dtype_code, lib, ptr, require_gpu, stream_ptr

MAX_SPLITS_CAP = 256
TOKENS_PER_SPLIT = 128


def _row_major_d(t: torch.Tensor, name: str) -> torch.Tensor:
    """Return ``t`` with a unit stride on the last dim and 16-byte aligned rows."""
    esz = t.element_size()
    vec = 16 // esz
    ok = (t.stride(-1) == 1 and t.data_ptr() % 16 == 0
          and all(s % vec == 0 for s in t.stride()[:-1]))
    return t if ok else t.contiguous()


class KVBlocks(NamedTuple):
    """A block pool layout of K/V: ``table`` [B, pages] int32 maps a
    sequence's page to a block of the pool [num_blocks, Hkv, page_size, D]
    (no counterpart in the reference, whose cache is contiguous)."""
    table: torch.Tensor
    num_blocks: int


class AppendRow(NamedTuple):
    """One row appended by the top-k step itself: k_new, v_new [B, Hkv, D]
    at row ``pos`` of every sequence, with the mean/std statistics views
    (min/max are the step's own k_min/k_max)."""
    k_new: torch.Tensor
    v_new: torch.Tensor
    k_mean: torch.Tensor
    k_std: torch.Tensor
    pos: int


def _bt_args(blocks: "KVBlocks | None"):
    if blocks is None:
        return (None, 0, 0)
    t = blocks.table
    if t.dtype != torch.int32 or t.dim() != 2 or t.stride(1) != 1 or not t.is_cuda:
        raise ValueError("block table must be a row-major int32 [B, pages] GPU tensor")
    return (t.data_ptr(), t.stride(0), int(blocks.num_blocks))


def choose_splits(max_tokens: int) -> int:
    """Workgroups per (b, kv head) for the decode kernels."""
    return int(max(1, min(MAX_SPLITS_CAP, math.ceil(max_tokens / TOKENS_PER_SPLIT))))


def qscale_for(alpha: float, head_dim: int, dtype: torch.dtype) -> float:
    """(alpha-1)/sqrt(D) rounded to the storage dtype (kernels/adadecode_paged.py:79,97,605)."""
    c = (alpha - 1.0) * (1.0 / math.sqrt(head_dim))
    return float(torch.tensor(c, dtype=torch.float64).to(dtype).to(torch.float64))


def page_quantile_z(quantile: float, page_size: int) -> float:
    """Normal quantile of quantile**(1/ps), as kernels/selection_pack.py:238-239."""
    return NormalDist().inv_cdf(quantile ** (1.0 / page_size))


# ---------------------------------------------------------------------------
# page statistics (kv_cache.py:40-116)
# ---------------------------------------------------------------------------

def page_stats(k: torch.Tensor, kmin, kmax, kmean, kstd, seq_len: int, page_size: int,
               page_begin: int, page_end: int, seq_lens: torch.Tensor | None = None) -> None:
    """Fill stats for pages [page_begin, page_end) from rows of k [B, Hkv, S_cap, D]
    (``seq_lens`` [B] int32: each sequence's pages end at its own length)."""
    require_gpu(k, kmin)
    B, Hkv, _, D = k.shape
    call("ekv_page_stats", k.data_ptr(), k.stride(0), k.stride(1), k.stride(2),
         kmin.data_ptr(), kmax.data_ptr(), kmean.data_ptr(), kstd.data_ptr(),
         kmin.stride(0), kmin.stride(1), kmin.stride(2), B, Hkv, D, seq_len, ptr(seq_lens),
         page_size, page_begin, page_end, dtype_code(k.dtype), stream_ptr(k.device))


def append_token(k_new, v_new, k, v, kmin, kmax, kmean, kstd, pos: int, page_size: int,
                 pos_per_batch: torch.Tensor | None = None,
                 blocks: KVBlocks | None = None) -> None:
    """Write row ``pos`` of K/V and recompute its page statistics, in place
    (``k``/``v`` the block pool when ``blocks`` is given)."""
    require_gpu(k_new, v_new, k)
    B, Hkv, D = kmin.shape[0], k.shape[1], k.shape[3]
    k_new = _row_major_d(k_new, "k_new")
    v_new = _row_major_d(v_new, "v_new")
    if k_new.stride() != v_new.stride():
        v_new = v_new.contiguous()
        k_new = k_new.contiguous()
    call("ekv_append", k_new.data_ptr(), v_new.data_ptr(), k_new.stride(0), k_new.stride(1),
         k.data_ptr(), v.data_ptr(), k.stride(0), k.stride(1), k.stride(2),
         kmin.data_ptr(), kmax.data_ptr(), kmean.data_ptr(), kstd.data_ptr(),
         kmin.stride(0), kmin.stride(1), kmin.stride(2), B, Hkv, D, pos,
         ptr(pos_per_batch), *_bt_args(blocks), page_size, dtype_code(k.dtype),
         stream_ptr(k.device))


# ---------------------------------------------------------------------------
# criticality + top-k (kernels/page_criticality.py, attention_topk.py:52-71)
# ---------------------------------------------------------------------------

def estimate_page_criticality(q, k_min, k_max, alibi_slopes=None, q_pos: int = 0,
                              page_size: int = 16, seq_len: int = 0,
                              exclude_last_page: bool = False, out: torch.Tensor | None = None,
                              topk: tuple | None = None,
                              seq_lens: torch.Tensor | None = None) -> torch.Tensor:
    """Upper-bound page scores [B, H, P(-1)] in the query dtype.

    Mirrors triton_estimate_page_criticality (kernels/page_criticality.py:107-187,
    apply_scaling=False).  ``topk=(k, last_page, page_indices)`` also produces
    the top-k page table (ekv_topk_pages semantics) in the same call.
    ``seq_lens`` [B] (ragged batch): sequence b scores, selects and appends its
    last page for its own length; the score rows keep the longest's stride.
    """
    require_gpu(q, k_min, k_max)
    B, H, _, D = q.shape
    _, Hkv, stored_pages, _ = k_min.shape
    num_pages = stored_pages - int(exclude_last_page)
    if num_pages < 0:
        raise ValueError("cannot exclude the last page from an empty cache")
    if out is None:
        out = torch.empty(B, H, num_pages, device=q.device, dtype=q.dtype)
    if num_pages == 0:
        return out
    if k_min.stride() != k_max.stride():
        raise ValueError("k_min and k_max must share strides")
    q3 = _row_major_d(q.reshape(B, H, D) if q.shape[2] == 1 else q[:, :, 0], "q")
    slopes = None
    if alibi_slopes is not None:
        slopes = alibi_slopes.to(device=q.device, dtype=torch.float32).contiguous()
    k_sel, last_page, pidx = (-1, -1, None) if topk is None else topk
    call("ekv_page_criticality", q3.data_ptr(), q3.stride(0), q3.stride(1),
         k_min.data_ptr(), k_max.data_ptr(), k_min.stride(0), k_min.stride(1), k_min.stride(2),
         ptr(slopes), out.data_ptr(), B, H, Hkv, D, num_pages, page_size, seq_len, q_pos,
         k_sel, last_page, ptr(seq_lens), ptr(pidx), 0 if pidx is None else pidx.stride(0),
         0 if pidx is None else pidx.stride(1), dtype_code(q.dtype),
         stream_ptr(q.device))
    return out


def topk_pages(scores: torch.Tensor, k: int, num_kv_heads: int, last_page: int = -1,
               out: torch.Tensor | None = None) -> torch.Tensor:
    """Top-k page table [B, Hkv, k (+1)] from scores [B, H, P] (ascending, ties to lower id)."""
    require_gpu(scores)
    B, H, P = scores.shape
    if not 0 <= k <= P:
        raise ValueError(f"k={k} out of range for {P} pages")
    width = k + (1 if last_page >= 0 else 0)
    if out is None:
        out = torch.empty(B, num_kv_heads, max(width, 1), device=scores.device, dtype=torch.int32)
    scores = scores.contiguous()
    call("ekv_topk_pages", scores.data_ptr(), B, H, num_kv_heads, P, k, last_page,
         out.data_ptr(), out.stride(0), out.stride(1), dtype_code(scores.dtype),
         stream_ptr(scores.device))
    return out


# ---------------------------------------------------------------------------
# paged decode (kernels/adadecode_paged.py:567-762, adadecode_paged_gaussian_tau.py)
# ---------------------------------------------------------------------------

class DecodeWorkspace:
    """Device workspace for one decode shape (score spill rows; needs no initialisation)."""

    def __init__(self, batch, nheads, num_kv_heads, dim, splits, max_tokens, device):
        self.spec = (batch, nheads, num_kv_heads, dim, splits, max_tokens, torch.device(device))
        nbytes = lib().ekv_decode_workspace_bytes(batch, nheads, num_kv_heads, dim, splits,
                                                  max_tokens)
        self.buf = torch.zeros(int(nbytes), dtype=torch.uint8, device=device)
        self.taus = torch.zeros(batch, nheads, dtype=torch.float32, device=device)
        self.splits = splits
        self.max_tokens = max_tokens


def _cache_seqlens_2d(cache_seqlens, batch, num_kv_heads):
    if cache_seqlens.dtype != torch.int32:
        cache_seqlens = cache_seqlens.to(torch.int32)
    if cache_seqlens.dim() == 1:
        cache_seqlens = cache_seqlens[:, None].expand(batch, num_kv_heads)
    assert tuple(cache_seqlens.shape) == (batch, num_kv_heads), "cache_seqlens must be [B, H_kv]"
    return cache_seqlens


def paged_entmax_decode(q, k_cache, v_cache, out, cache_seqlens, page_indices, page_size,
                        alpha, tau_mode: int, iters: int, tau: torch.Tensor | None,
                        alibi_slopes=None, q_seqlens=None, workspace: DecodeWorkspace | None = None,
                        kv_rows: int | None = None, tau_in: torch.Tensor | None = None,
                        blocks: KVBlocks | None = None):
    """Shared launcher of the exact-tau (tau_mode 0) and given-tau (1) decode.

    The final tau goes to ``tau`` (the workspace's buffer when None); in
    given-tau mode the start value is read from ``tau_in`` (default: ``tau``).
    With ``blocks``, ``k_cache``/``v_cache`` are the block pool
    [num_blocks, Hkv, page_size, D] and ``kv_rows`` bounds a sequence's rows.
    """
    require_gpu(q, k_cache, v_cache, out, page_indices)
    batch, nheads, q_len, dim = q.shape
    num_kv_heads = k_cache.shape[1]
    assert q_len == 1
    assert page_indices.dtype == torch.int32
    assert nheads % num_kv_heads == 0, "Query heads must be divisible by KV heads"
    assert tuple(v_cache.shape) == tuple(k_cache.shape), "K/V cache shapes must match"
    if blocks is None:
        assert k_cache.shape[0] == batch, "K/V cache batch mismatch"
    assert page_indices.shape[0] == batch, "page_indices batch mismatch"
    assert page_indices.shape[1] == num_kv_heads, "page_indices must be keyed by KV heads"
    if k_cache.stride() != v_cache.stride():
        raise ValueError("k_cache and v_cache must share strides")
    if k_cache.dtype != q.dtype or v_cache.dtype != q.dtype:
        raise TypeError("q, k_cache and v_cache must share a dtype")
    cache_seqlens = _cache_seqlens_2d(cache_seqlens, batch, num_kv_heads)
    if page_indices.stride(2) != 1:
        page_indices = page_indices.contiguous()
    n_slots = page_indices.shape[2]
    max_tokens = n_slots * page_size
    if workspace is None:
        workspace = DecodeWorkspace(batch, nheads, num_kv_heads, dim, choose_splits(max_tokens),
                                    max_tokens, q.device)
    elif workspace.spec[:4] != (batch, nheads, num_kv_heads, dim) or workspace.max_tokens < max_tokens:
        raise ValueError(f"invalid paged workspace {workspace.spec} for shape "
                         f"{(batch, nheads, num_kv_heads, dim, max_tokens)}")
    if tau is None:
        tau = workspace.taus
    assert tuple(tau.shape) == (batch, nheads) and tau.dtype == torch.float32 and tau.is_contiguous(), \
        "tau must be a contiguous float32 [B, H] tensor"
    if tau_mode == 1:
        if tau_in is None:
            tau_in = tau
        assert tuple(tau_in.shape) == (batch, nheads) and tau_in.dtype == torch.float32 \
            and tau_in.is_contiguous(), "tau_in must be a contiguous float32 [B, H] tensor"
    q3 = _row_major_d(q[:, :, 0], "q")
    o3 = out[:, :, 0]
    direct = o3.stride(-1) == 1 and o3.data_ptr() % 16 == 0
    o_target = o3 if direct else torch.empty(batch, nheads, dim, device=q.device, dtype=q.dtype)
    slopes = None
    if alibi_slopes is not None:
        slopes = alibi_slopes.to(device=q.device, dtype=torch.float32).contiguous()
    qsl = None
    if q_seqlens is not None:
        qsl = q_seqlens.to(device=q.device, dtype=torch.int32).contiguous()
    if kv_rows is None:
        kv_rows = k_cache.shape[2] if blocks is None else blocks.table.shape[1] * page_size
    call("ekv_paged_entmax_decode",
         q3.data_ptr(), q3.stride(0), q3.stride(1), k_cache.data_ptr(), v_cache.data_ptr(),
         k_cache.stride(0), k_cache.stride(1), k_cache.stride(2), kv_rows, *_bt_args(blocks),
         page_indices.data_ptr(), page_indices.stride(0), page_indices.stride(1), n_slots,
         cache_seqlens.data_ptr(), cache_seqlens.stride(0), cache_seqlens.stride(1),
         ptr(qsl), ptr(slopes), ptr(tau_in), tau.data_ptr(), tau_mode, iters,
         o_target.data_ptr(), o_target.stride(0), o_target.stride(1), float(alpha),
         qscale_for(alpha, dim, q.dtype), page_size, batch, nheads, num_kv_heads, dim,
         workspace.splits, workspace.max_tokens, workspace.buf.data_ptr(),
         workspace.buf.numel(), dtype_code(q.dtype), stream_ptr(q.device))
    if not direct:
        o3.copy_(o_target)
    return out


def topk_paged_entmax_decode(q, k_min, k_max, scores, k_select: int, last_page: int,
                             k_cache, v_cache, out, page_indices, cache_seqlens, page_size: int,
                             alpha: float, niter: int, seq_len: int, q_pos: int,
                             alibi_slopes=None, q_seqlens=None,
                             workspace: DecodeWorkspace | None = None, kv_rows: int | None = None,
                             taus_out: torch.Tensor | None = None,
                             blocks: KVBlocks | None = None,
                             seq_lens: torch.Tensor | None = None,
                             append: AppendRow | None = None):
    """Criticality + top-k + exact-tau decode of one step (ekv_topk_paged_entmax_decode).

    Scores the pages [0, scores.shape[2]) into ``scores``, writes the top-k page
    table (last page at slot k) into ``page_indices`` [B, Hkv, k + 1] and the
    decode output into ``out``; a single launch when the shape allows it.
    With ``append`` the row is appended first, inside the same launch when it
    is fused (ekv_append_topk_paged_entmax_decode; uniform batches only).
    """
    require_gpu(q, k_min, k_max, scores, k_cache, v_cache, out, page_indices)
    batch, nheads, q_len, dim = q.shape
    num_kv_heads = k_cache.shape[1]
    assert q_len == 1
    assert nheads % num_kv_heads == 0, "Query heads must be divisible by KV heads"
    num_pages = scores.shape[2]
    if not 1 <= k_select <= num_pages:
        raise ValueError(f"k={k_select} out of range for {num_pages} pages")
    if k_min.stride() != k_max.stride():
        raise ValueError("k_min and k_max must share strides")
    if k_cache.stride() != v_cache.stride():
        raise ValueError("k_cache and v_cache must share strides")
    if k_cache.dtype != q.dtype or v_cache.dtype != q.dtype or scores.dtype != q.dtype:
        raise TypeError("q, scores, k_cache and v_cache must share a dtype")
    assert scores.is_contiguous() and tuple(scores.shape[:2]) == (batch, nheads)
    n_slots = k_select + (1 if last_page >= 0 else 0)
    assert page_indices.dtype == torch.int32 and page_indices.stride(2) == 1
    assert tuple(page_indices.shape) == (batch, num_kv_heads, n_slots), "page_indices shape"
    cache_seqlens = _cache_seqlens_2d(cache_seqlens, batch, num_kv_heads)
    max_tokens = n_slots * page_size
    if workspace is None:
        workspace = DecodeWorkspace(batch, nheads, num_kv_heads, dim, choose_splits(max_tokens),
                                    max_tokens, q.device)
    elif workspace.spec[:4] != (batch, nheads, num_kv_heads, dim) or workspace.max_tokens < max_tokens:
        raise ValueError(f"invalid paged workspace {workspace.spec} for shape "
                         f"{(batch, nheads, num_kv_heads, dim, max_tokens)}")
    tau = workspace.taus if taus_out is None else taus_out
    assert tuple(tau.shape) == (batch, nheads) and tau.dtype == torch.float32 and tau.is_contiguous()
    q3 = _row_major_d(q[:, :, 0], "q")
    o3 = out[:, :, 0]
    direct = o3.stride(-1) == 1 and o3.data_ptr() % 16 == 0
    o_target = o3 if direct else torch.empty(batch, nheads, dim, device=q.device, dtype=q.dtype)
    slopes = None
    if alibi_slopes is not None:
        slopes = alibi_slopes.to(device=q.device, dtype=torch.float32).contiguous()
    qsl = None
    if q_seqlens is not None:
        qsl = q_seqlens.to(device=q.device, dtype=torch.int32).contiguous()
    if kv_rows is None:
        kv_rows = k_cache.shape[2] if blocks is None else blocks.table.shape[1] * page_size
    head = ()
    name = "ekv_topk_paged_entmax_decode"
    if append is not None:
        if seq_lens is not None:
            raise ValueError("a fused append needs a uniform batch")
        kn = _row_major_d(append.k_new, "k_new")
        vn = _row_major_d(append.v_new, "v_new")
        if kn.stride() != vn.stride():
            kn, vn = kn.contiguous(), vn.contiguous()
        if append.k_mean.stride() != k_min.stride() or append.k_std.stride() != k_min.stride():
            raise ValueError("k_mean and k_std must share k_min's strides")
        head = (kn.data_ptr(), vn.data_ptr(), kn.stride(0), kn.stride(1),
                append.k_mean.data_ptr(), append.k_std.data_ptr(), int(append.pos))
        name = "ekv_append_topk_paged_entmax_decode"
    call(name, *head,
         q3.data_ptr(), q3.stride(0), q3.stride(1), k_min.data_ptr(), k_max.data_ptr(),
         k_min.stride(0), k_min.stride(1), k_min.stride(2), scores.data_ptr(), num_pages,
         seq_len, q_pos, k_select, last_page, k_cache.data_ptr(), v_cache.data_ptr(),
         k_cache.stride(0), k_cache.stride(1), k_cache.stride(2), kv_rows, *_bt_args(blocks),
         page_indices.data_ptr(), page_indices.stride(0), page_indices.stride(1),
         cache_seqlens.data_ptr(), cache_seqlens.stride(0), cache_seqlens.stride(1),
         ptr(qsl), ptr(slopes), ptr(seq_lens), tau.data_ptr(), niter, o_target.data_ptr(),
         o_target.stride(0),
         o_target.stride(1), float(alpha), qscale_for(alpha, dim, q.dtype), page_size, batch,
         nheads, num_kv_heads, dim, workspace.splits, workspace.max_tokens,
         workspace.buf.data_ptr(), workspace.buf.numel(), dtype_code(q.dtype),
         stream_ptr(q.device))
    if not direct:
        o3.copy_(o_target)
    return out


def sparse_attention_decode_paged(q, k_cache, v_cache, out, cache_seqlens, page_indices,
                                  page_size, alibi_slopes=None, is_causal=True, alpha=1.5,
                                  niter=10, max_splits=32, bins=16, q_seqlens=None,
                                  taus_out=None, workspace=None):
    """Exact-tau paged decode; mirrors kernels/adadecode_paged.py:567-762.

    ``max_splits`` is accepted for signature parity; the split count is chosen
    from the page table width (or taken from ``workspace``).  ``bins`` must be 16.
    """
    if bins != 16:
        raise ValueError("only 16 histogram bins are supported")
    paged_entmax_decode(q, k_cache, v_cache, out, cache_seqlens, page_indices, page_size, alpha,
                        0, niter, taus_out, alibi_slopes, q_seqlens, workspace)
    return out


def sparse_attention_decode_paged_gaussian_tau(q, k_cache, v_cache, out, cache_seqlens,
                                               page_indices, page_size, tau, alibi_slopes=None,
                                               alpha=1.5, max_splits=32, q_seqlens=None,
                                               tau_correction_iters=0, workspace=None):
    """Given-tau paged decode; mirrors kernels/adadecode_paged_gaussian_tau.py:192-331.

    ``tau`` [B, H] float32 is updated in place with the corrected value.
    """
    batch, nheads = q.shape[:2]
    assert tuple(tau.shape) == (batch, nheads), "tau must be [B, H]"
    paged_entmax_decode(q, k_cache, v_cache, out, cache_seqlens, page_indices, page_size, alpha,
                        1, tau_correction_iters, tau, alibi_slopes, q_seqlens, workspace)
    return out


# ---------------------------------------------------------------------------
# dense (non-paged) decode (kernels/adadecode.py:754-1016)
# ---------------------------------------------------------------------------

class DenseDecodeWorkspace:
    """Device workspace of the dense decode for one (B, H, kv_rows) shape."""

    def __init__(self, batch, nheads, kv_rows, device):
        self.spec = (batch, nheads, kv_rows, torch.device(device))
        nbytes = lib().ekv_dense_decode_workspace_bytes(batch, nheads, kv_rows)
        if nbytes < 0:
            raise ValueError(f"unsupported dense decode shape {self.spec[:3]}")
        self.buf = torch.empty(int(nbytes), dtype=torch.uint8, device=device)


def sparse_attention_decode_orchestrator(q, k_cache, v_cache, out, cache_seqlens,
                                         token_positions, alibi_slopes=None,
                                         is_causal: bool = True, alpha: float = 1.5,
                                         niter: int = 10, max_splits: int = 32, bins: int = 16,
                                         q_seqlens=None, profile: dict | None = None,
                                         workspace: DenseDecodeWorkspace | None = None,
                                         taus_out: torch.Tensor | None = None):
    """Dense alpha-entmax decode over a contiguous cache (kernels/adadecode.py:754-1016).

    q [B, H, 1, D]; k_cache, v_cache [B, Hkv, S, D] (the reference requires
    Hkv == H; H a multiple of Hkv is accepted here); cache_seqlens [B]: head
    (b, h) attends to keys [0, cache_seqlens[b]).  token_positions [B, Hkv, S]
    (int) give the keys' positions for ALiBi, and the query sits at
    q_seqlens[b] - 1 (q_seqlens defaults to cache_seqlens, :787-791).  tau is
    the 16-bin histogram init plus ``niter`` bracketed Halley steps, as the
    reference's stages 1-5; the output is the unnormalised weighted sum of
    stages 6a/6b.  ``is_causal`` has no effect in the reference's kernels
    (the causal masks are commented out, :530, :696-697) nor here;
    ``max_splits`` is the reference's launch width and does not change
    results here (the native launch sizes itself); only ``bins == 16`` is
    supported.  ``profile`` (a dict) accumulates the step's device time in
    ms under "total" and counts calls under "_count", as the reference's
    per-stage dict does (:1008-1012); the step is one native launch sequence
    so per-stage keys do not exist.
    """
    require_gpu(q, k_cache, v_cache, out, cache_seqlens)
    batch, nheads, q_len, dim = q.shape
    assert q_len == 1
    num_kv_heads = k_cache.shape[1]
    assert k_cache.shape[0] == batch, f"k_cache batch mismatch: {k_cache.shape[0]} != {batch}"
    assert nheads % num_kv_heads == 0, "Query heads must be divisible by KV heads"
    assert k_cache.shape[3] == dim, f"k_cache dim mismatch: {k_cache.shape[3]} != {dim}"
    assert tuple(v_cache.shape) == tuple(k_cache.shape), "k_cache and v_cache shapes differ"
    if bins != 16:
        raise ValueError(f"bins={bins}: the native histogram init has 16 bins")
    if niter < 0:
        raise ValueError(f"niter must be >= 0 (got {niter})")
    if k_cache.dtype != q.dtype or v_cache.dtype != q.dtype:
        raise TypeError("q, k_cache and v_cache must share a dtype")
    kv_rows = k_cache.shape[2]
    k = _row_major_d(k_cache, "k_cache")
    v = _row_major_d(v_cache, "v_cache")
    if k.stride() != v.stride():
        v = v.contiguous()
        k = k.contiguous()
    q3 = _row_major_d(q[:, :, 0], "q")
    o3 = out[:, :, 0]
    direct = o3.stride(-1) == 1 and o3.data_ptr() % 16 == 0
    o_target = o3 if direct else torch.empty(batch, nheads, dim, device=q.device, dtype=q.dtype)
    csl = cache_seqlens.to(device=q.device, dtype=torch.int32).contiguous()
    assert tuple(csl.shape) == (batch,), "cache_seqlens must be [B]"
    slopes = _alibi_f32(alibi_slopes, q.device)
    pos = None
    if slopes is not None and token_positions is not None:
        pos = token_positions.to(device=q.device, dtype=torch.int32)
        assert tuple(pos.shape) == (batch, num_kv_heads, kv_rows), \
            "token_positions must be [B, H_kv, S]"
        if pos.stride(-1) != 1:
            pos = pos.contiguous()
    qsl = None
    if slopes is not None:
        qsl = (q_seqlens if q_seqlens is not None else cache_seqlens)
        qsl = qsl.to(device=q.device, dtype=torch.int32).contiguous()
    if workspace is None or workspace.spec != (batch, nheads, kv_rows, q.device):
        workspace = DenseDecodeWorkspace(batch, nheads, kv_rows, q.device)
    taus = taus_out if taus_out is not None else torch.empty(batch, nheads, dtype=torch.float32,
                                                             device=q.device)
    assert tuple(taus.shape) == (batch, nheads) and taus.dtype == torch.float32 \
        and taus.is_contiguous(), "taus_out must be a contiguous float32 [B, H] tensor"
    events = None
    if profile is not None:
        events = (torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
        events[0].record()
    call("ekv_dense_entmax_decode",
         q3.data_ptr(), q3.stride(0), q3.stride(1), k.data_ptr(), v.data_ptr(), k.stride(0),
         k.stride(1), k.stride(2), kv_rows, csl.data_ptr(), ptr(pos),
         0 if pos is None else pos.stride(0), 0 if pos is None else pos.stride(1), ptr(qsl),
         ptr(slopes), taus.data_ptr(), int(niter), o_target.data_ptr(), o_target.stride(0),
         o_target.stride(1), float(alpha), qscale_for(alpha, dim, q.dtype), batch, nheads,
         num_kv_heads, dim, workspace.buf.data_ptr(), workspace.buf.numel(), dtype_code(q.dtype),
         stream_ptr(q.device))
    if not direct:
        o3.copy_(o_target)
    if events is not None:
        events[1].record()
        torch.cuda.synchronize(q.device)
        profile["total"] = profile.get("total", 0.0) + events[0].elapsed_time(events[1])
        profile["_count"] = profile.get("_count", 0) + 1
    return out


# ---------------------------------------------------------------------------
# Gaussian statistics, tau solvers, selection (gaussian_page_stats.py, tau_solver_gpu.py,
# tau_mixture_solver_triton.py, selection_pack.py, tau_clamp.py)
# ---------------------------------------------------------------------------

class GaussianBuffers:
    """Persistent outputs + zero-initialised workspace of the Gaussian stats launch."""

    def __init__(self, batch, nheads, num_kv_heads, dim, pages, dtype, device):
        f = dict(dtype=torch.float32, device=device)
        self.spec = (batch, nheads, num_kv_heads, dim, pages, dtype, torch.device(device))
        self.mu_p = torch.empty(batch, nheads, pages, **f)
        self.sigma_p = torch.empty(batch, nheads, pages, **f)
        self.mu_g = torch.empty(batch, nheads, 1, **f)
        self.sigma_g = torch.empty(batch, nheads, 1, **f)
        self.mean_var = torch.empty(batch, nheads, 1, **f)
        self.var_means = torch.empty(batch, nheads, 1, **f)
        self.tau_hat = torch.empty(batch, nheads, **f)
        nbytes = lib().ekv_gaussian_workspace_bytes(batch, nheads, num_kv_heads, dim, pages,
                                                    dtype_code(dtype))
        self.ws = torch.zeros(int(nbytes), dtype=torch.uint8, device=device)


def compute_page_gaussian_stats(q, k_mean, k_std, pages_for_stats, *, alibi_slopes=None,
                                page_size=16, seq_len=0, alpha=1.5, n_tokens=None,
                                solve_tau=True, tau_iters=120, tol=1e-6,
                                buffers: GaussianBuffers | None = None,
                                seq_lens: torch.Tensor | None = None) -> GaussianBuffers:
    """Per-page score moments, global moments and (optionally) the fused tau-hat.

    Mirrors compute_page_gaussian_stats_triton (kernels/gaussian_page_stats.py:128-233,
    return_sigma=True) plus gaussian_utils.py:142-181.  ``n_tokens`` defaults to
    pages_for_stats * page_size (seq_len_for_stats).
    """
    require_gpu(q, k_mean, k_std)
    if q.shape[0] != k_mean.shape[0] or q.shape[1] % k_mean.shape[1] != 0:
        raise ValueError("q and k_mean must have matching batch/head dimensions")
    if k_mean.shape != k_std.shape or k_mean.stride() != k_std.stride():
        raise ValueError("k_mean and k_std must have identical shapes")
    if pages_for_stats <= 0:
        raise ValueError("pages_for_stats must be positive")
    if pages_for_stats > k_mean.shape[2]:
        raise ValueError("pages_for_stats exceeds the available pages")
    if q.shape[-1] != k_mean.shape[-1]:
        raise ValueError("q and page statistics must have matching head dimensions")
    B, H, _, D = q.shape
    Hkv = k_mean.shape[1]
    if buffers is None or buffers.spec != (B, H, Hkv, D, pages_for_stats, q.dtype, q.device):
        buffers = GaussianBuffers(B, H, Hkv, D, pages_for_stats, q.dtype, q.device)
    if n_tokens is None:
        n_tokens = pages_for_stats * page_size
    q3 = _row_major_d(q[:, :, 0], "q")
    slopes = None
    if alibi_slopes is not None:
        slopes = alibi_slopes.to(device=q.device, dtype=torch.float32)
        if slopes.dim() == 2:
            slopes = slopes[0]
        slopes = slopes.contiguous()
    call("ekv_gaussian_page_stats", q3.data_ptr(), q3.stride(0), q3.stride(1),
         k_mean.data_ptr(), k_std.data_ptr(), k_mean.stride(0), k_mean.stride(1),
         k_mean.stride(2), pages_for_stats, ptr(slopes), page_size, seq_len,
         buffers.mu_p.data_ptr(), buffers.sigma_p.data_ptr(), buffers.mu_g.data_ptr(),
         buffers.sigma_g.data_ptr(), buffers.mean_var.data_ptr(), buffers.var_means.data_ptr(),
         buffers.tau_hat.data_ptr() if solve_tau else None, float(alpha), int(n_tokens),
         int(tau_iters), float(tol), ptr(seq_lens), B, H, Hkv, D, buffers.ws.data_ptr(),
         buffers.ws.numel(),
         dtype_code(q.dtype), stream_ptr(q.device))
    return buffers


def _alibi_f32(alibi_slopes, device):
    if alibi_slopes is None:
        return None
    slopes = alibi_slopes.to(device=device, dtype=torch.float32)
    if slopes.dim() == 2:
        slopes = slopes[0]
    return slopes.contiguous()


def compute_page_gaussian_moments(q, k_mean, k_std, pages_for_stats, buffers: GaussianBuffers, *,
                                  alibi_slopes=None, page_size=16, seq_len=0,
                                  n_tokens=None,
                                  seq_lens: torch.Tensor | None = None) -> GaussianBuffers:
    """Per-page moments mu_p / sigma_p and the partial sums of the global moments
    (the first launch of the Gaussian step; kernels/gaussian_page_stats.py:8-121)."""
    require_gpu(q, k_mean, k_std)
    B, H, _, D = q.shape
    Hkv = k_mean.shape[1]
    if buffers.spec != (B, H, Hkv, D, pages_for_stats, q.dtype, q.device):
        raise ValueError(f"Gaussian buffers {buffers.spec} do not match the step")
    if k_mean.stride() != k_std.stride():
        raise ValueError("k_mean and k_std must share strides")
    if n_tokens is None:
        n_tokens = pages_for_stats * page_size
    q3 = _row_major_d(q[:, :, 0], "q")
    call("ekv_gaussian_moments", q3.data_ptr(), q3.stride(0), q3.stride(1), k_mean.data_ptr(),
         k_std.data_ptr(), k_mean.stride(0), k_mean.stride(1), k_mean.stride(2), pages_for_stats,
         ptr(_alibi_f32(alibi_slopes, q.device)), page_size, seq_len, int(n_tokens),
         ptr(seq_lens), buffers.mu_p.data_ptr(), buffers.sigma_p.data_ptr(), B, H, Hkv, D, buffers.ws.data_ptr(),
         buffers.ws.numel(), dtype_code(q.dtype), stream_ptr(q.device))
    return buffers


def gaussian_paged_entmax_decode(q, k_cache, v_cache, out, buffers: GaussianBuffers, *,
                                 pages_for_stats: int, num_pages: int, n_tokens: int,
                                 page_size: int, alpha: float, tau_hat_given: bool,
                                 safety_margin_z, max_quantile,
                                 threshold_excess_margin_fraction: float, page_indices, counts,
                                 tau_floor, cache_seqlens, last_page_size: int, tau_clamped,
                                 clamp_quantile: float, effective, tau_out, tau_mode: int,
                                 iters: int, workspace: DecodeWorkspace, alibi_slopes=None,
                                 q_seqlens=None, kv_rows=None, eps: float = 1e-4,
                                 tau_iters: int = 120, tol: float = 1e-6,
                                 seq_lens: torch.Tensor | None = None,
                                 blocks: KVBlocks | None = None):
    """Selection + decode of one Gaussian-aware step after compute_page_gaussian_moments
    (ekv_gaussian_paged_entmax_decode): global moments and tau-hat (unless
    ``tau_hat_given``), threshold select + pack + clamp (``tau_clamped`` None =
    no clamp), then the given-tau (tau_mode 1) or exact (0) decode."""
    require_gpu(q, k_cache, v_cache, out, page_indices)
    B, H, _, D = q.shape
    Hkv = k_cache.shape[1]
    if k_cache.stride() != v_cache.stride():
        raise ValueError("k_cache and v_cache must share strides")
    if k_cache.dtype != q.dtype or v_cache.dtype != q.dtype:
        raise TypeError("q, k_cache and v_cache must share a dtype")
    assert page_indices.dtype == torch.int32 and page_indices.stride(2) == 1
    assert tuple(page_indices.shape) == (B, Hkv, num_pages), "page_indices shape"
    max_tokens = num_pages * page_size
    if workspace.spec[:4] != (B, H, Hkv, D) or workspace.max_tokens < max_tokens:
        raise ValueError(f"invalid paged workspace {workspace.spec}")
    auto = safety_margin_z is None or max_quantile is None
    z_page = page_quantile_z(max_quantile, page_size) if not auto else 0.0
    smz = float(safety_margin_z) if not auto else 0.0
    q3 = _row_major_d(q[:, :, 0], "q")
    o3 = out[:, :, 0]
    direct = o3.stride(-1) == 1 and o3.data_ptr() % 16 == 0
    o_target = o3 if direct else torch.empty(B, H, D, device=q.device, dtype=q.dtype)
    qsl = None if q_seqlens is None else q_seqlens.to(device=q.device, dtype=torch.int32).contiguous()
    if kv_rows is None:
        kv_rows = k_cache.shape[2] if blocks is None else blocks.table.shape[1] * page_size
    call("ekv_gaussian_paged_entmax_decode",
         buffers.ws.data_ptr(), buffers.ws.numel(), buffers.mu_p.data_ptr(),
         buffers.sigma_p.data_ptr(), pages_for_stats, num_pages, buffers.mu_g.data_ptr(),
         buffers.sigma_g.data_ptr(), buffers.mean_var.data_ptr(), buffers.var_means.data_ptr(),
         buffers.tau_hat.data_ptr(), int(bool(tau_hat_given)), int(n_tokens), int(tau_iters),
         float(tol), int(auto), smz, z_page, page_quantile_z(0.99, page_size),
         page_quantile_z(0.995, page_size), float(threshold_excess_margin_fraction),
         page_indices.data_ptr(), page_indices.stride(0), page_indices.stride(1),
         counts.data_ptr(), tau_floor.data_ptr(), cache_seqlens.data_ptr(), int(last_page_size),
         ptr(tau_clamped), page_quantile_z(clamp_quantile, page_size), float(eps), ptr(effective),
         q3.data_ptr(), q3.stride(0), q3.stride(1), k_cache.data_ptr(), v_cache.data_ptr(),
         k_cache.stride(0), k_cache.stride(1), k_cache.stride(2), kv_rows, *_bt_args(blocks),
         ptr(qsl),
         ptr(_alibi_f32(alibi_slopes, q.device)), ptr(seq_lens), tau_out.data_ptr(),
         int(tau_mode), int(iters),
         o_target.data_ptr(), o_target.stride(0), o_target.stride(1), float(alpha),
         qscale_for(alpha, D, q.dtype), page_size, B, H, Hkv, D, workspace.max_tokens,
         workspace.buf.data_ptr(), workspace.buf.numel(), dtype_code(q.dtype),
         stream_ptr(q.device))
    if not direct:
        o3.copy_(o_target)
    return out


def solve_for_tau_hat_single_gaussian_gpu(mu_g, sigma_g, n, alpha, iterations=120, tol=1e-6,
                                          out=None):
    """One lane per (b, h) tau-hat; mirrors kernels/tau_solver_gpu.py:128-158."""
    require_gpu(mu_g, sigma_g)
    shape = mu_g.shape
    mu = mu_g.contiguous().view(-1).to(torch.float32)
    sg = sigma_g.contiguous().view(-1).to(torch.float32)
    res = torch.empty_like(mu) if out is None else out.view(-1)
    call("ekv_tau_single_gaussian", mu.data_ptr(), sg.data_ptr(), res.data_ptr(), mu.numel(),
         int(n), float(alpha), int(iterations), float(tol), stream_ptr(mu.device))
    return res.view(shape)


def solve_for_tau_hat_page_gaussian_mixture(mu_pages, sigma_pages, page_counts=None, alpha=1.5,
                                            max_iter=40, tol=1e-6, uniform_page_count=1.0,
                                            seq_lens=None, page_size=16):
    """Page-mixture tau-hat [..., 1]; mirrors kernels/tau_mixture_solver_triton.py:172-240.

    Per-page counts other than one uniform value are not supported by the
    native kernel (the reference path only passes a uniform count,
    gaussian_utils.py:171-177).
    """
    if mu_pages.shape != sigma_pages.shape:
        raise ValueError(f"mu_pages and sigma_pages must have the same shape, got "
                         f"{tuple(mu_pages.shape)} and {tuple(sigma_pages.shape)}")
    if mu_pages.dim() < 1:
        raise ValueError("mu_pages must have a page dimension")
    if alpha not in (2, 1.5, 4 / 3):
        raise ValueError(f"Unsupported alpha for page-mixture tau solve: {alpha}")
    if page_counts is not None:
        pc = torch.as_tensor(page_counts)
        if pc.numel() != 1 and not bool((pc == pc.reshape(-1)[0]).all()):
            raise ValueError("non-uniform page_counts are not supported")
        uniform_page_count = float(pc.reshape(-1)[0])
    if uniform_page_count <= 0:
        raise ValueError("uniform_page_count must be positive")
    require_gpu(mu_pages, sigma_pages)
    pages = mu_pages.shape[-1]
    if pages <= 0:
        raise ValueError("mu_pages must have a non-empty page dimension")
    rows = mu_pages.numel() // pages
    mu = mu_pages.to(torch.float32).contiguous()
    sg = sigma_pages.to(torch.float32).contiguous()
    out = torch.empty(rows, device=mu.device, dtype=torch.float32)
    call("ekv_tau_page_mixture", mu.data_ptr(), sg.data_ptr(), out.data_ptr(), rows, pages,
         float(uniform_page_count), float(alpha), int(max_iter), float(tol), ptr(seq_lens),
         int(mu_pages.shape[1]) if (seq_lens is not None and mu_pages.dim() >= 3) else 1,
         int(page_size), stream_ptr(mu.device))
    return out.view(*mu_pages.shape[:-1], 1).to(mu_pages.dtype)


def select_gaussian_threshold_pack(mu_p, sigma_p, tau_hat, sigma_g, page_size, alpha,
                                   safety_margin_z, max_quantile,
                                   threshold_excess_margin_fraction, pages_for_stats, num_pages,
                                   num_kv_heads=None, out=None, counts=None, tau_floor=None,
                                   cache_seqlens=None, last_page_size=None, tau_clamped=None,
                                   clamp_quantile=0.5, eps=1e-4, effective=None, seq_lens=None):
    """Threshold select + pack (+ fused lengths and tau clamp).

    Mirrors select_gaussian_threshold_pack_triton (kernels/selection_pack.py:201-272).
    ``safety_margin_z``/``max_quantile`` None selects the automatic margins of
    gaussian_utils.py:163-169, computed on the device.
    Returns (page_indices [B, Hkv, num_pages], counts [B, Hkv], tau_floor [B, H]).
    """
    require_gpu(mu_p, sigma_p, tau_hat, sigma_g)
    if mu_p.dim() != 3:
        raise ValueError("mu_scores_per_page must have shape [batch, heads, pages]")
    if pages_for_stats <= 0 or num_pages <= 0:
        raise ValueError("pages_for_stats and num_pages must be positive")
    B, H, _ = mu_p.shape
    Hkv = H if num_kv_heads is None else num_kv_heads
    dev = mu_p.device
    if out is None:
        out = torch.empty(B, Hkv, num_pages, dtype=torch.int32, device=dev)
    if counts is None:
        counts = torch.empty(B, Hkv, dtype=torch.int32, device=dev)
    if tau_floor is None:
        tau_floor = torch.empty(B, H, dtype=torch.float32, device=dev)
    th = tau_hat.reshape(B, H).to(torch.float32).contiguous()
    sg = sigma_g.reshape(B, H).to(torch.float32).contiguous()
    auto = safety_margin_z is None or max_quantile is None
    z_low = page_quantile_z(0.99, page_size)
    z_high = page_quantile_z(0.995, page_size)
    z_page = page_quantile_z(max_quantile, page_size) if not auto else 0.0
    smz = float(safety_margin_z) if not auto else 0.0
    z_clamp = page_quantile_z(clamp_quantile, page_size)
    if last_page_size is None:
        last_page_size = page_size
    call("ekv_select_gaussian_pack", mu_p.contiguous().data_ptr(), sigma_p.contiguous().data_ptr(),
         th.data_ptr(), sg.data_ptr(), B, H, Hkv, pages_for_stats, num_pages, float(alpha),
         int(auto), smz, z_page, z_low, z_high, float(threshold_excess_margin_fraction),
         out.data_ptr(), out.stride(0), out.stride(1), counts.data_ptr(), tau_floor.data_ptr(),
         ptr(cache_seqlens), page_size, last_page_size, ptr(tau_clamped), z_clamp, float(eps),
         ptr(effective), ptr(seq_lens), stream_ptr(dev))
    return out, counts, tau_floor


def clamp_tau_to_selected_page_statistics(tau, mu_p, sigma_p, page_indices, num_selected,
                                          tau_floor, page_size, alpha, clamp_quantile,
                                          pages_for_stats, eps=1e-4):
    """Standalone tau clamp; mirrors kernels/tau_clamp.py:76-151."""
    require_gpu(tau, mu_p, sigma_p, page_indices, num_selected)
    if pages_for_stats <= 0:
        return tau.contiguous()
    original_shape = tau.shape
    t2 = tau.squeeze(-1) if tau.dim() == 3 and tau.shape[-1] == 1 else tau
    B, H = t2.shape
    t2 = t2.to(torch.float32).contiguous()
    if page_indices.shape[-1] <= 0:
        out = t2.clone()
        return out.unsqueeze(-1) if original_shape != out.shape else out
    Hsel = page_indices.shape[1]
    pi = page_indices if page_indices.stride(-1) == 1 else page_indices.contiguous()
    tf = None
    if tau_floor is not None:
        tf = tau_floor.squeeze(-1) if tau_floor.dim() == 3 and tau_floor.shape[-1] == 1 else tau_floor
        tf = tf.to(device=t2.device, dtype=torch.float32).contiguous()
    out = torch.empty_like(t2)
    ns = num_selected.to(torch.int32)
    call("ekv_tau_clamp", t2.data_ptr(), mu_p.contiguous().data_ptr(),
         sigma_p.contiguous().data_ptr(), pi.data_ptr(), pi.stride(0), pi.stride(1),
         pi.shape[-1], ns.data_ptr(), ns.stride(0), ns.stride(1), ptr(tf), out.data_ptr(), B, H,
         Hsel, pages_for_stats, float(alpha), page_quantile_z(clamp_quantile, page_size),
         float(eps), stream_ptr(t2.device))
    if original_shape != out.shape:
        out = out.unsqueeze(-1)
    return out


def cache_seqlens_from_page_counts(counts, page_size, last_page_size, out=None):
    """max(count-1, 0)*ps + last_page_size; mirrors kernels/selection_pack.py:23-43."""
    require_gpu(counts)
    c = counts.to(torch.int32).contiguous()
    if out is None:
        out = torch.empty_like(c)
    call("ekv_cache_seqlens_from_counts", c.data_ptr(), out.data_ptr(), c.numel(), page_size,
         last_page_size, stream_ptr(c.device))
    return out
