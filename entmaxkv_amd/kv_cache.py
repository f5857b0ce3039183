"""Paged KV cache with per-page key statistics, MI355X layout.

Drop-in for ``entmaxkv.kv_cache.PagedKVCache`` (kv_cache.py:16-255): same
constructor, methods and attributes.  What changes is the storage:

* K and V live in preallocated capacity buffers ``[B, Hkv, S_cap, D]``;
  ``k_cache``/``v_cache`` are views of the first ``seq_len`` rows.  ``append``
  writes one row in place (one kernel launch that also refreshes the last
  page's statistics) instead of ``torch.cat`` of the whole cache
  (kv_cache.py:81-82), and capacity grows geometrically when full.
* The four statistics are interleaved per page: ``bounds [B, Hkv, P_cap, 2, D]``
  holds (min, max) and ``moments [B, Hkv, P_cap, 2, D]`` holds (mean, std), so
  the criticality kernel reads one contiguous 2*D run per page and the
  Gaussian kernel another.  ``k_min``/``k_max``/``k_mean``/``k_std`` are views
  ``[B, Hkv, P, D]`` of them.
* ``initialize`` computes all page statistics with one kernel launch instead
  of a Python loop over pages (kv_cache.py:58-70).
* Ragged batches (no counterpart in the reference, whose cache holds one
  length): ``initialize(k, v, seq_lens=...)`` gives every sequence its own
  length.  ``seq_lens`` (device int32 [B]) then drives every kernel: each
  sequence has its own pages, last page, statistics and append position;
  ``seq_len`` is the longest length and fixes the buffer shapes.
* Block pool (no counterpart in the reference either): with
  ``block_pool=True`` K and V live in a pool ``[num_blocks, Hkv, page_size,
  D]`` shared by the batch, and a block table (device int32 [B, pages])
  maps page p of sequence b to its block.  Blocks are handed out from a free
  list as pages fill (page-major over the batch, so the sequences' blocks
  interleave in the pool), the statistics stay per sequence, and every kernel
  reads K/V through the table.  ``k_cache``/``v_cache`` then gather a
  contiguous copy.
"""

from __future__ import annotations

from collections import deque
from typing import Optional

import torch

from . import kernels as K


def _round_up(x: int, m: int) -> int:
    return (x + m - 1) // m * m


class PagedKVCache:
    """KV cache with paged min/max/mean/std metadata (kv_cache.py:16-38)."""

    def __init__(self, page_size: int = 16, capacity: Optional[int] = None,
                 headroom: int = 1024, block_pool: bool = False,
                 num_blocks: Optional[int] = None):
        self.page_size = page_size
        self.capacity = capacity
        self.headroom = headroom
        self.block_pool = block_pool
        self.num_blocks = num_blocks  # pool size (default: every sequence's capacity)
        self._table = None  # device int32 [B, pages cap] (block pool)
        self._table_host = None
        self._free = None
        self._batch = 0
        self.seq_len = 0
        self.seq_lens: Optional[torch.Tensor] = None  # [B] int32 on the device (ragged batch)
        self._lens_host = None
        self._k = None
        self._v = None
        self._bounds = None
        self._moments = None

        self.last_num_selected_per_head = None
        self.last_effective_safety_margin = None
        self.last_effective_max_quantile = None
        self.last_page_scores = None

        self._page_indices_buf: Optional[torch.Tensor] = None
        self._page_indices_last_page: Optional[int] = None
        self._scores_buf: Optional[torch.Tensor] = None
        self._paged_decode_workspaces: dict = {}
        self._gaussian_buffers: dict = {}
        self._select_buffers: dict = {}

    # ------------------------------------------------------------------ views
    @property
    def num_pages(self) -> int:
        return (self.seq_len + self.page_size - 1) // self.page_size

    def _gather_pool(self, pool):
        """Contiguous [B, Hkv, seq_len, D] copy of a block pool's rows."""
        P = self.num_pages
        blocks = self._table[:, :P].long().clamp(min=0)  # unassigned pages read block 0
        g = pool[blocks]  # [B, P, Hkv, ps, D]
        B, _, Hkv, ps, D = g.shape
        return g.permute(0, 2, 1, 3, 4).reshape(B, Hkv, P * ps, D)[:, :, : self.seq_len]

    @property
    def k_cache(self):
        if self._k is None:
            return None
        return self._gather_pool(self._k) if self.block_pool else self._k[:, :, : self.seq_len]

    @property
    def v_cache(self):
        if self._v is None:
            return None
        return self._gather_pool(self._v) if self.block_pool else self._v[:, :, : self.seq_len]

    @property
    def num_kv_heads(self) -> int:
        return self._k.shape[1]

    @property
    def block_table(self) -> Optional[torch.Tensor]:
        """Device int32 [B, pages cap] (block pool only; -1 = no block yet)."""
        return self._table

    def kv_operands(self):
        """(k, v, kv_rows, blocks) as the decode launchers take them: the
        capacity buffers [B, Hkv, cap, D], or the pool with its table."""
        if self.block_pool:
            return (self._k, self._v, self._table.shape[1] * self.page_size,
                    K.KVBlocks(self._table, self._k.shape[0]))
        return self._k, self._v, self._k.shape[2], None

    def _stat(self, buf, j):
        return None if buf is None else buf[:, :, : self.num_pages, j]

    @property
    def k_min(self):
        return self._stat(self._bounds, 0)

    @property
    def k_max(self):
        return self._stat(self._bounds, 1)

    @property
    def k_mean(self):
        return self._stat(self._moments, 0)

    @property
    def k_std(self):
        return self._stat(self._moments, 1)

    @property
    def is_ragged(self) -> bool:
        return self.seq_lens is not None

    def compacted_seqlens(self, token_budget: int) -> torch.Tensor:
        """Per-sequence compacted token counts of a top-k step, [B] int32 on the
        device: min(budget // ps, P_b - 1) * ps + last_page_size_b (what the
        reference's caller passes as ``cache_seqlens``, tests/test_topk.py:81-85)."""
        ps = self.page_size
        lens = self.seq_lens if self.seq_lens is not None else torch.full(
            (self._batch,), self.seq_len, dtype=torch.int32, device=self._k.device)
        pages = (lens + ps - 1) // ps
        k = torch.clamp(pages - 1, min=0, max=token_budget // ps)
        return (k * ps + lens - (pages - 1) * ps).to(torch.int32)

    @property
    def kv_capacity(self) -> int:
        if self._k is None:
            return 0
        return self._table.shape[1] * self.page_size if self.block_pool else self._k.shape[2]

    # ------------------------------------------------------------- storage
    def _allocate(self, batch, num_heads, cap, head_dim, dtype, device):
        cap = _round_up(max(cap, self.page_size), self.page_size)
        pcap = cap // self.page_size
        k = torch.empty(batch, num_heads, cap, head_dim, dtype=dtype, device=device)
        v = torch.empty_like(k)
        bounds = torch.zeros(batch, num_heads, pcap, 2, head_dim, dtype=dtype, device=device)
        moments = torch.zeros_like(bounds)
        return k, v, bounds, moments

    def _grow(self, needed: int):
        if self.block_pool:
            self._grow_table(_round_up(max(needed, 2 * self.kv_capacity), self.page_size)
                             // self.page_size)
            return
        B, H, cap, D = self._k.shape
        new_cap = max(needed, 2 * cap)
        k, v, bounds, moments = self._allocate(B, H, new_cap, D, self._k.dtype, self._k.device)
        k[:, :, :cap].copy_(self._k)
        v[:, :, :cap].copy_(self._v)
        pc = self._bounds.shape[2]
        bounds[:, :, :pc].copy_(self._bounds)
        moments[:, :, :pc].copy_(self._moments)
        self._k, self._v, self._bounds, self._moments = k, v, bounds, moments

    # ------------------------------------------------------------- block pool
    def _grow_table(self, pcap: int):
        """Widen the block table (and the statistics) to ``pcap`` pages."""
        B, old = self._table_host.shape
        table = torch.full((B, pcap), -1, dtype=torch.int32)
        table[:, :old] = self._table_host
        self._table_host = table
        self._table = table.to(self._k.device)
        H, D = self._bounds.shape[1], self._bounds.shape[4]
        bounds = torch.zeros(B, H, pcap, 2, D, dtype=self._k.dtype, device=self._k.device)
        moments = torch.zeros_like(bounds)
        bounds[:, :, :old].copy_(self._bounds)
        moments[:, :, :old].copy_(self._moments)
        self._bounds, self._moments = bounds, moments

    def _take_block(self) -> int:
        if not self._free:
            # pool exhausted: double it (block ids stay valid)
            n = self._k.shape[0]
            k = torch.empty((2 * n,) + tuple(self._k.shape[1:]), dtype=self._k.dtype,
                            device=self._k.device)
            v = torch.empty_like(k)
            k[:n].copy_(self._k)
            v[:n].copy_(self._v)
            self._k, self._v = k, v
            self._free.extend(range(n, 2 * n))
        return self._free.popleft()

    def _init_pool(self, k, v, seq_len, cap):
        B, H, _, D = k.shape
        ps = self.page_size
        pcap = _round_up(max(cap, ps), ps) // ps
        nblocks = self.num_blocks if self.num_blocks is not None else B * pcap
        P = (seq_len + ps - 1) // ps
        lens = self._lens_host if self._lens_host is not None else torch.full((B,), seq_len)
        pages = (lens + ps - 1) // ps
        if int(pages.sum()) > nblocks:
            raise ValueError(f"num_blocks={nblocks} cannot hold {int(pages.sum())} pages")
        self._k = torch.empty(nblocks, H, ps, D, dtype=k.dtype, device=k.device)
        self._v = torch.empty_like(self._k)
        self._bounds = torch.zeros(B, H, pcap, 2, D, dtype=k.dtype, device=k.device)
        self._moments = torch.zeros_like(self._bounds)
        self._free = deque(range(nblocks))
        table = torch.full((B, pcap), -1, dtype=torch.int32)
        for p in range(P):  # page-major: the sequences' blocks interleave
            for b in range(B):
                if p < int(pages[b]):
                    table[b, p] = self._free.popleft()
        self._table_host = table
        self._table = table.to(k.device)
        if P == 0:
            return None
        # page-padded contiguous copy: the statistics source and the scatter source
        kp = torch.zeros(B, H, P * ps, D, dtype=k.dtype, device=k.device)
        vp = torch.zeros_like(kp)
        kp[:, :, :seq_len].copy_(k[:, :, :seq_len])
        vp[:, :, :seq_len].copy_(v[:, :, :seq_len])
        valid = table[:, :P] >= 0
        idx = table[:, :P][valid].long().to(k.device)
        vd = valid.to(k.device)
        self._k.index_copy_(0, idx, kp.view(B, H, P, ps, D).permute(0, 2, 1, 3, 4)[vd])
        self._v.index_copy_(0, idx, vp.view(B, H, P, ps, D).permute(0, 2, 1, 3, 4)[vd])
        return kp

    def _assign_append_blocks(self, pos: int):
        """Give every sequence whose next row opens a page a block for it."""
        ps = self.page_size
        lens = self._lens_host if self._lens_host is not None else torch.full(
            (self._batch,), pos, dtype=torch.int64)
        need = int(lens.max()) // ps + 1
        if need > self._table_host.shape[1]:
            self._grow_table(max(need, 2 * self._table_host.shape[1]))
        changed = False
        for b in range(self._batch):
            page = int(lens[b]) // ps
            if self._table_host[b, page] < 0:
                self._table_host[b, page] = self._take_block()
                changed = True
        if changed:
            self._table.copy_(self._table_host)

    def initialize(self, k: torch.Tensor, v: torch.Tensor, seq_lens=None):
        """Initialize the cache with prefill keys/values (kv_cache.py:40-70).

        ``seq_lens`` (optional, [B] ints): sequence b holds only its first
        seq_lens[b] rows of ``k``/``v`` (a ragged batch).
        """
        if not k.is_cuda:
            raise ValueError("PagedKVCache requires GPU tensors")
        batch, num_heads, seq_len, head_dim = k.shape
        self.seq_lens = None
        self._lens_host = None
        if seq_lens is not None:
            host = torch.as_tensor(seq_lens, dtype=torch.int64).reshape(-1).cpu().clone()
            if host.numel() != batch:
                raise ValueError(f"seq_lens has {host.numel()} entries for a batch of {batch}")
            if bool((host < 1).any()) or bool((host > seq_len).any()):
                raise ValueError(f"seq_lens must lie in [1, {seq_len}]")
            self._lens_host = host
            self.seq_lens = host.to(device=k.device, dtype=torch.int32)
            seq_len = int(host.max())
        cap = self.capacity if self.capacity is not None else seq_len + self.headroom
        cap = max(cap, seq_len + 1)
        self._batch = batch
        if self.block_pool:
            src = self._init_pool(k, v, seq_len, cap)
        else:
            self._k, self._v, self._bounds, self._moments = self._allocate(
                batch, num_heads, cap, head_dim, k.dtype, k.device)
            self._k[:, :, :seq_len].copy_(k[:, :, :seq_len])
            self._v[:, :, :seq_len].copy_(v[:, :, :seq_len])
            src = self._k
        self.seq_len = seq_len
        self._page_indices_buf = None
        self._page_indices_last_page = None
        if seq_len > 0:
            K.page_stats(src, self._bounds[:, :, :, 0], self._bounds[:, :, :, 1],
                         self._moments[:, :, :, 0], self._moments[:, :, :, 1], seq_len,
                         self.page_size, 0, self.num_pages, seq_lens=self.seq_lens)

    def append(self, k_new: torch.Tensor, v_new: torch.Tensor):
        """Append one token per (b, kv head) and update its page's stats (kv_cache.py:72-116).

        k_new, v_new: [batch, num_heads, 1, head_dim].
        """
        if k_new.shape[2] != 1:
            for t in range(k_new.shape[2]):
                self.append(k_new[:, :, t:t + 1], v_new[:, :, t:t + 1])
            return
        pos = self.seq_len
        blocks = None
        if self.block_pool:
            self._assign_append_blocks(pos)
            blocks = K.KVBlocks(self._table, self._k.shape[0])
        elif pos + 1 > self.kv_capacity:
            self._grow(pos + 1 + self.headroom)
        K.append_token(k_new[:, :, 0], v_new[:, :, 0], self._k, self._v,
                       self._bounds[:, :, :, 0], self._bounds[:, :, :, 1],
                       self._moments[:, :, :, 0], self._moments[:, :, :, 1], pos, self.page_size,
                       pos_per_batch=self.seq_lens, blocks=blocks)
        if self.seq_lens is not None:
            # every sequence grows by one token at its own position
            self.seq_lens.add_(1)
            self._lens_host += 1
            self.seq_len = int(self._lens_host.max())
        else:
            self.seq_len = pos + 1

    def reserve_append(self, k_new: torch.Tensor, v_new: torch.Tensor) -> "K.AppendRow":
        """The host side of ``append`` for a uniform batch and one token: the
        row is reserved (capacity, block), ``seq_len`` counts it, and the
        returned row is written by the next top-k step's launch
        (``kernels.topk_paged_entmax_decode(append=...)``) or by
        ``write_append``."""
        if self.seq_lens is not None or k_new.shape[2] != 1:
            raise ValueError("reserve_append: uniform batch and one token only")
        pos = self.seq_len
        if self.block_pool:
            self._assign_append_blocks(pos)
        elif pos + 1 > self.kv_capacity:
            self._grow(pos + 1 + self.headroom)
        self.seq_len = pos + 1
        return K.AppendRow(k_new[:, :, 0], v_new[:, :, 0], self._moments[:, :, :, 0],
                           self._moments[:, :, :, 1], pos)

    def write_append(self, row: "K.AppendRow") -> None:
        """Writes a row reserved by ``reserve_append`` with its own launch."""
        blocks = K.KVBlocks(self._table, self._k.shape[0]) if self.block_pool else None
        K.append_token(row.k_new, row.v_new, self._k, self._v, self._bounds[:, :, :, 0],
                       self._bounds[:, :, :, 1], row.k_mean, row.k_std, row.pos,
                       self.page_size, blocks=blocks)

    # ---------------------------------------------------------- criticality
    def estimate_page_criticality(self, q: torch.Tensor, use_triton: bool = False,
                                  alibi_slopes=None, q_pos: int = 0,
                                  exclude_last_page: bool = False) -> torch.Tensor:
        """Upper-bound page scores [B, H, pages] (kv_cache.py:118-165).

        ``use_triton`` is accepted for compatibility; the native kernel always runs.
        """
        return K.estimate_page_criticality(
            q, self.k_min, self.k_max, alibi_slopes=alibi_slopes, q_pos=q_pos,
            page_size=self.page_size, seq_len=self.seq_len,
            exclude_last_page=exclude_last_page,
            seq_lens=self.seq_lens if exclude_last_page else None)

    def select_topk(self, q: torch.Tensor, k: int, alibi_slopes=None) -> torch.Tensor:
        """Fused criticality + top-k page table [B, Hkv, k + 1] (last page at slot k).

        Replaces attention_topk.py:45-71.  Under GQA a kv head takes the k
        pages of best rank over its query heads' own page orders (ties to the
        lower page index).  In a ragged batch sequence b
        selects k_b = min(k, P_b - 1) pages, its last page at slot k_b.
        """
        B, H = q.shape[:2]
        Hkv = self._k.shape[1]
        P = self.num_pages
        last = P - 1
        buf = self.get_page_indices_buf(B, Hkv, k, last)
        scores = self._get_scores_buf(B, H, P - 1, q.dtype, q.device)
        self.last_page_scores = scores
        if k == 0:
            if self.seq_lens is not None:
                # every sequence's own last page
                last_b = (self.seq_lens + self.page_size - 1) // self.page_size - 1
                buf[:, :, 0].copy_(last_b[:, None].expand(B, Hkv))
            return buf
        K.estimate_page_criticality(
            q, self.k_min, self.k_max, alibi_slopes=alibi_slopes, q_pos=self.seq_len - 1,
            page_size=self.page_size, seq_len=self.seq_len, exclude_last_page=True,
            out=scores, topk=(k, last, buf), seq_lens=self.seq_lens)
        return buf

    def _get_scores_buf(self, B, H, P, dtype, device):
        buf = self._scores_buf
        need = B * H * max(P, 1)
        if buf is None or buf.numel() < need or buf.dtype != dtype or buf.device != device:
            buf = torch.empty(max(need, 2 * need), dtype=dtype, device=device)
            self._scores_buf = buf
        return buf[: B * H * P].view(B, H, P)

    # ---------------------------------------------------------- buffers
    def get_page_indices_buf(self, batch: int, num_heads: int, num_pages_to_select: int,
                             last_page_idx: int) -> torch.Tensor:
        """Persistent [B, H, n_selected+1] page-index buffer (kv_cache.py:167-185).

        The sentinel column is written by the selection kernel on every call, so
        no per-step fill is needed; it is filled here only when nothing is
        selected.
        """
        target_shape = (batch, num_heads, num_pages_to_select + 1)
        buf = self._page_indices_buf
        device = self._k.device
        if buf is None or tuple(buf.shape) != target_shape or buf.device != device:
            buf = torch.empty(target_shape, dtype=torch.int32, device=device)
            self._page_indices_buf = buf
            self._page_indices_last_page = None
        if num_pages_to_select == 0 and self._page_indices_last_page != last_page_idx:
            buf[:, :, 0].fill_(last_page_idx)
        self._page_indices_last_page = last_page_idx
        return buf

    def get_paged_decode_workspace(self, batch: int, nheads: int, dim: int, max_splits: int,
                                   bins: int, dtype: torch.dtype, device, *,
                                   num_kv_heads: Optional[int] = None,
                                   max_tokens: Optional[int] = None) -> K.DecodeWorkspace:
        """Persistent decode workspace for one shape (kv_cache.py:187-203).

        ``max_splits`` and ``bins`` are accepted for signature parity; the split
        count follows from ``max_tokens`` (the page-table width times page size).
        """
        device = torch.device(device)
        if num_kv_heads is None:
            num_kv_heads = self._k.shape[1]
        if max_tokens is None:
            max_tokens = self.num_pages * self.page_size
        splits = K.choose_splits(max_tokens)
        key = (batch, nheads, num_kv_heads, dim, splits, max_tokens, device.type, device.index)
        ws = self._paged_decode_workspaces.get(key)
        if ws is None:
            ws = K.DecodeWorkspace(batch, nheads, num_kv_heads, dim, splits, max_tokens, device)
            self._paged_decode_workspaces[key] = ws
        return ws

    def get_gaussian_buffers(self, q: torch.Tensor, pages_for_stats: int) -> K.GaussianBuffers:
        B, H, _, D = q.shape
        key = (B, H, self._k.shape[1], D, pages_for_stats, q.dtype, q.device)
        buf = self._gaussian_buffers.get(key)
        if buf is None:
            self._gaussian_buffers.clear()
            buf = K.GaussianBuffers(B, H, self._k.shape[1], D, pages_for_stats, q.dtype, q.device)
            self._gaussian_buffers[key] = buf
        return buf

    def _get_select_buffers(self, B, H, Hkv, num_pages, device):
        key = (B, H, Hkv, num_pages, device)
        sb = self._select_buffers.get(key)
        if sb is None:
            self._select_buffers.clear()
            sb = {
                "page_indices": torch.zeros(B, Hkv, num_pages, dtype=torch.int32, device=device),
                "counts": torch.zeros(B, Hkv, dtype=torch.int32, device=device),
                "tau_floor": torch.zeros(B, H, dtype=torch.float32, device=device),
                "cache_seqlens": torch.zeros(B, Hkv, dtype=torch.int32, device=device),
                "tau_clamped": torch.zeros(B, H, dtype=torch.float32, device=device),
                "effective": torch.zeros(2, dtype=torch.float32, device=device),
            }
            self._select_buffers[key] = sb
        return sb

    # ---------------------------------------------------------- Gaussian selection
    def select_gaussian_aware(self, q: torch.Tensor, alpha: float = 1.5,
                              safety_margin_z: float = 0.0, max_quantile: float = 0.99,
                              gaussian_stats: dict = None, clamp: bool = False,
                              last_page_size: Optional[int] = None):
        """Gaussian threshold selection + pack (kv_cache.py:205-255).

        As in the reference, ``safety_margin_z``/``max_quantile`` arguments are
        superseded by the values in ``gaussian_stats`` (None there = automatic,
        derived on the device from the mean sigma_global).  Returns
        (page_indices [B, Hkv, P], num_selected [B, Hkv]); slots beyond the count
        are unspecified.  Also fills gaussian_stats["tau_floor"], and, with
        ``clamp``, gaussian_stats["tau_clamped"] and
        gaussian_stats["cache_seqlens"].
        """
        st = gaussian_stats
        B, H = q.shape[:2]
        Hkv = self._k.shape[1]
        num_pages = st["num_pages"]
        pfs = st["pages_for_stats"]
        sb = self._get_select_buffers(B, H, Hkv, num_pages, q.device)
        frac = st.get("threshold_excess_margin_fraction", 0.1)
        if last_page_size is None:
            last_page_size = self.page_size
        K.select_gaussian_threshold_pack(
            st["mu_scores_per_page"], st["sigma_scores_per_page"], st["tau_hat"],
            st["sigma_global"], self.page_size, alpha, st["safety_margin_z"], st["max_quantile"],
            float(frac), pfs, num_pages, num_kv_heads=Hkv, out=sb["page_indices"],
            counts=sb["counts"], tau_floor=sb["tau_floor"], cache_seqlens=sb["cache_seqlens"],
            last_page_size=last_page_size, tau_clamped=sb["tau_clamped"] if clamp else None,
            clamp_quantile=st.get("tau_clamp_page_max_quantile", 0.5), effective=sb["effective"])
        self.record_gaussian_selection(st, sb, clamp)
        return sb["page_indices"], sb["counts"]

    def record_gaussian_selection(self, st: dict, sb: dict, clamp: bool) -> None:
        """Publish a Gaussian selection's buffers in the stats dict and on the cache."""
        st["tau_floor"] = sb["tau_floor"]
        st["cache_seqlens"] = sb["cache_seqlens"]
        if clamp:
            st["tau_clamped"] = sb["tau_clamped"]
        st["effective_margins"] = sb["effective"]
        self.last_effective_safety_margin = (
            sb["effective"][0] if st["safety_margin_z"] is None else st["safety_margin_z"])
        self.last_effective_max_quantile = (
            sb["effective"][1] if st["max_quantile"] is None else st["max_quantile"])
        self.last_num_selected_per_head = sb["counts"]
