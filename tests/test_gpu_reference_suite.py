"""The reference's own accuracy suites on this build (tests/test_topk.py and
tests/test_gaussian.py of deep-spin/entmaxkv): the same shapes, seeds,
coverages, thresholds and latency bar, against the same oracle -- dense
entmax attention computed on the GPU (fp32 scores, row-wise entmax,
tests/benchmark_utils.py:56-83), here with this build's `triton_entmax`,
whose own parity with the CPU oracle is checked in tests/test_gpu_dense.py.

The inputs are i.i.d. normal, so the reference's thresholds are loose by
design (tests/test_gaussian.py:26): these tests show the drop-in runs the
reference's cases within the reference's bars; the exact parity of every
stage is checked in tests/test_gpu_parity.py.
"""

from __future__ import annotations

import math
import time

import pytest
import torch

pytestmark = pytest.mark.gpu

TOPK_BATCHES = [1, 8]
TOPK_KV_LENS = [1024, 2048, 8192, 16384, 64000]
TOPK_COVERAGES = [0.25, 0.50]
TOPK_ALPHAS = [1.5, 2.0]
DTYPES = {"fp16": torch.float16, "fp32": torch.float32}
GAUSSIAN_BATCHES = [1, 8]
GAUSSIAN_KV_LENS = [2048, 8192, 16384, 64000]


def _case(**kw):
    print("CASE", " ".join(f"{k}={v}" for k, v in kw.items()), flush=True)


def alibi_slopes(n_heads: int) -> torch.Tensor:
    """Half the heads linear ALiBi slopes, half 0 (tests/benchmark_utils.py:24-31)."""
    half = n_heads // 2
    a = torch.exp2(-8 * torch.arange(1, half + 1, device="cuda") / half)
    return torch.cat([a, torch.zeros(half, device="cuda")]).float()


def reference_attention(q, k, v, alpha, alibi=None):
    """Dense entmax attention (tests/benchmark_utils.py:56-83): fp32 scores /
    sqrt(D), ALiBi slope * (k_pos - q_pos), row-wise entmax, p @ v."""
    from entmaxkv_amd.entmax import triton_entmax
    B, H, q_len, D = q.shape
    kv_len = k.shape[2]
    qk = torch.matmul(q.float(), k.float().transpose(-1, -2)) / math.sqrt(D)
    if alibi is not None:
        qp = torch.arange(kv_len - q_len, kv_len, device=q.device)
        kp = torch.arange(kv_len, device=q.device)
        diff = (kp[None, :] - qp[:, None]).float()
        qk = qk + alibi.view(1, H, 1, 1) * diff.view(1, 1, q_len, kv_len)
    p = triton_entmax(qk.contiguous(), alpha=alpha, n_iter=2, fast_math=True)
    return torch.matmul(p, v.float()).to(q.dtype)


def rel_error(ref, out):
    """||ref - out|| / ||ref|| (tests/benchmark_utils.py:38-49)."""
    return float(torch.norm(ref.float() - out.float()) / torch.norm(ref.float()))


def latency_ms(fn, warmup=3, iters=10):
    for _ in range(warmup):
        fn()
        torch.cuda.synchronize()
    ts = []
    for _ in range(iters):
        t0 = time.perf_counter()
        fn()
        torch.cuda.synchronize()
        ts.append((time.perf_counter() - t0) * 1e3)
    return sorted(ts)[len(ts) // 2]


def run_topk(seed, batch, kv_len, coverage, alpha, use_alibi, dtype, kv_heads=8, q_heads=8,
             head_dim=64, page_size=16):
    """tests/test_topk.py:37-157 (run_topk_benchmark)."""
    from entmaxkv_amd import PagedKVCache, sparse_attention_decode_paged
    torch.manual_seed(seed)
    torch.cuda.manual_seed_all(seed)
    dev = torch.device("cuda")
    alibi = alibi_slopes(q_heads) if use_alibi else None
    page_budget = max(1, int((coverage * kv_len + page_size - 1) // page_size))
    token_budget = page_budget * page_size
    k_full = torch.randn(batch, kv_heads, kv_len, head_dim, device=dev, dtype=dtype)
    v_full = torch.randn(batch, kv_heads, kv_len, head_dim, device=dev, dtype=dtype)
    q = torch.randn(batch, q_heads, 1, head_dim, device=dev, dtype=dtype)
    k_new = torch.randn(batch, kv_heads, 1, head_dim, device=dev, dtype=dtype)
    v_new = torch.randn(batch, kv_heads, 1, head_dim, device=dev, dtype=dtype)
    n_rep = q_heads // kv_heads
    k_ref = torch.cat([k_full, k_new], 2).repeat_interleave(n_rep, 1)
    v_ref = torch.cat([v_full, v_new], 2).repeat_interleave(n_rep, 1)
    out_ref = reference_attention(q, k_ref, v_ref, alpha, alibi)
    full = kv_len + 1
    total_pages = (full + page_size - 1) // page_size
    n_sel = min(token_budget // page_size, total_pages - 1)
    eff = n_sel * page_size + full - (total_pages - 1) * page_size
    cache_seqlens = torch.full((batch,), eff, device=dev, dtype=torch.int32)
    q_seqlens = torch.full((batch,), full, device=dev, dtype=torch.int32)
    out = torch.zeros_like(q)
    cache = PagedKVCache(page_size=page_size)
    cache.initialize(k_full, v_full)
    cache.append(k_new, v_new)

    def call():
        sparse_attention_decode_paged(q=q, kv_cache=cache, k_new=k_new, v_new=v_new, out=out,
                                      token_budget=token_budget, cache_seqlens=cache_seqlens,
                                      q_seqlens=q_seqlens, alibi_slopes=alibi, alpha=alpha,
                                      niter=2, append_cache=False)

    lat = latency_ms(call)
    call()
    torch.cuda.synchronize()
    return rel_error(out_ref, out), lat


def run_gaussian(seed, batch, kv_len, tau_mode, use_alibi, dtype, kv_heads=8, q_heads=8,
                 head_dim=64, page_size=16):
    """tests/test_gaussian.py:37-135 (run_gaussian_benchmark): alpha 1.5,
    safety_margin_z 0.0, max_quantile 0.995."""
    from entmaxkv_amd import PagedKVCache, sparse_attention_decode_gaussian_aware_entmax
    torch.manual_seed(seed)
    torch.cuda.manual_seed_all(seed)
    dev = torch.device("cuda")
    alibi = alibi_slopes(q_heads) if use_alibi else None
    q = torch.randn(batch, kv_heads, 1, head_dim, device=dev, dtype=dtype)
    k_full = torch.randn(batch, kv_heads, kv_len, head_dim, device=dev, dtype=dtype)
    v_full = torch.randn(batch, kv_heads, kv_len, head_dim, device=dev, dtype=dtype)
    if q_heads != kv_heads:
        q = q.repeat_interleave(q_heads // kv_heads, dim=1)
    k_new = torch.randn(batch, kv_heads, 1, head_dim, device=dev, dtype=dtype)
    v_new = torch.randn(batch, kv_heads, 1, head_dim, device=dev, dtype=dtype)
    q_seqlens = torch.full((batch,), kv_len + 1, device=dev, dtype=torch.int32)
    out = torch.zeros_like(q)
    cache = PagedKVCache(page_size=page_size)
    cache.initialize(k_full, v_full)
    cache.append(k_new, v_new)

    def call():
        sparse_attention_decode_gaussian_aware_entmax(
            q=q, kv_cache=cache, k_new=k_new, v_new=v_new, out=out, alpha=1.5,
            safety_margin_z=0.0, max_quantile=0.995, alibi_slopes=alibi, append_cache=False,
            tau_mode=tau_mode, q_seqlens=q_seqlens)

    lat = latency_ms(call)
    call()
    torch.cuda.synchronize()
    n_rep = q_heads // kv_heads
    k_ref = torch.cat([k_full, k_new], 2).repeat_interleave(n_rep, 1)
    v_ref = torch.cat([v_full, v_new], 2).repeat_interleave(n_rep, 1)
    out_ref = reference_attention(q, k_ref, v_ref, 1.5, alibi)
    return rel_error(out_ref, out), lat


@pytest.mark.parametrize("dtype", list(DTYPES))
@pytest.mark.parametrize("alpha", TOPK_ALPHAS)
@pytest.mark.parametrize("batch", TOPK_BATCHES)
@pytest.mark.parametrize("kv_len", TOPK_KV_LENS)
@pytest.mark.parametrize("coverage", TOPK_COVERAGES)
def test_topk_paged_basic(batch, kv_len, coverage, alpha, dtype):
    """tests/test_topk.py:164-182."""
    _case(test="ref_topk_basic", batch=batch, kv_len=kv_len, coverage=coverage, alpha=alpha,
          dtype=dtype)
    err, lat = run_topk(1, batch, kv_len, coverage, alpha, False, DTYPES[dtype])
    print(f"rel_error {err:.4f} latency_ms {lat:.3f}", flush=True)
    assert err < (1.0 - coverage) * 2.0, f"rel_error {err:.4f}"
    assert lat < 500.0


@pytest.mark.parametrize("dtype", list(DTYPES))
@pytest.mark.parametrize("alpha", TOPK_ALPHAS)
@pytest.mark.parametrize("batch", TOPK_BATCHES)
@pytest.mark.parametrize("kv_len", TOPK_KV_LENS)
@pytest.mark.parametrize("coverage", TOPK_COVERAGES)
def test_topk_alibi(batch, kv_len, coverage, alpha, dtype):
    """tests/test_topk.py:184-201."""
    _case(test="ref_topk_alibi", batch=batch, kv_len=kv_len, coverage=coverage, alpha=alpha,
          dtype=dtype)
    err, lat = run_topk(2, batch, kv_len, coverage, alpha, True, DTYPES[dtype])
    print(f"rel_error {err:.4f} latency_ms {lat:.3f}", flush=True)
    assert err < (1.0 - coverage) * 2.0, f"rel_error {err:.4f}"


# (test name, seed, tau_mode, alibi, bar) -- tests/test_gaussian.py:158-214
GAUSSIAN_CASES = [("exact_basic", 10, "exact", False, 0.5),
                  ("corrected_basic", 12, "corrected", False, 0.5),
                  ("corrected_alibi", 12, "corrected", True, 0.5),
                  ("exact_alibi", 13, "exact", True, 0.6)]


@pytest.mark.parametrize("name,seed,tau_mode,alibi,bar", GAUSSIAN_CASES,
                         ids=[c[0] for c in GAUSSIAN_CASES])
@pytest.mark.parametrize("dtype", list(DTYPES))
@pytest.mark.parametrize("batch", GAUSSIAN_BATCHES)
@pytest.mark.parametrize("kv_len", GAUSSIAN_KV_LENS)
def test_gaussian(batch, kv_len, dtype, name, seed, tau_mode, alibi, bar):
    _case(test=f"ref_gaussian_{name}", batch=batch, kv_len=kv_len, dtype=dtype)
    err, lat = run_gaussian(seed, batch, kv_len, tau_mode, alibi, DTYPES[dtype])
    print(f"rel_error {err:.4f} latency_ms {lat:.3f}", flush=True)
    assert err < bar, f"rel_error {err:.4f}"
    if name in ("exact_basic",):
        assert lat < 500.0
