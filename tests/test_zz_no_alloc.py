"""ekv_topk_paged_entmax_decode_noalloc (static device scratch, no allocation)
against ekv_topk_paged_entmax_decode with a caller workspace, through the C ABI.

Two calls in a row on the split path (whose scores go through the workspace,
i.e. the scratch), the second smaller; then the fused path; then a step too
large for the scratch, rejected before any launch.  The kernels are the same,
so results must be bit-identical.
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from tests.gpu_helpers import TORCH_DT, randn, to_dev

pytestmark = pytest.mark.gpu


def _case(B, Hkv, G, pages, k_sel, dtype, seed):
    from entmaxkv_amd import PagedKVCache
    rng = np.random.default_rng(seed)
    ps, D = 16, 128
    S = pages * ps + 5
    H = Hkv * G
    cache = PagedKVCache(page_size=ps)
    cache.initialize(to_dev(randn(rng, (B, Hkv, S, D), dtype), dtype),
                     to_dev(randn(rng, (B, Hkv, S, D), dtype), dtype))
    q = to_dev(randn(rng, (B, H, 1, D), dtype), dtype)
    P = cache.num_pages
    return dict(cache=cache, q=q, B=B, H=H, Hkv=Hkv, D=D, ps=ps, S=S, P=P, k=k_sel,
                lps=S - (P - 1) * ps, dtype=dtype)


def _run(c, noalloc):
    """One step through the C ABI; returns (out, page table, tau, scores)."""
    from entmaxkv_amd import _lib
    from entmaxkv_amd.kernels import choose_splits, qscale_for
    dev = c["q"].device
    B, H, Hkv, D, ps, P, k = c["B"], c["H"], c["Hkv"], c["D"], c["ps"], c["P"], c["k"]
    cache = c["cache"]
    dt = TORCH_DT[c["dtype"]]
    n_slots = k + 1
    max_tokens = n_slots * ps
    splits = choose_splits(max_tokens)
    scores = torch.full((B, H, P - 1), 7.0, dtype=dt, device=dev)
    pidx = torch.full((B, Hkv, n_slots), -5, dtype=torch.int32, device=dev)
    seqlens = torch.full((B, Hkv), k * ps + c["lps"], dtype=torch.int32, device=dev)
    tau = torch.full((B, H), 9.0, dtype=torch.float32, device=dev)
    out = torch.full((B, H, D), 3.0, dtype=dt, device=dev)
    q3 = c["q"][:, :, 0]
    kmin, kmax, kc, vc = cache.k_min, cache.k_max, cache.k_cache, cache.v_cache
    args = [q3.data_ptr(), q3.stride(0), q3.stride(1), kmin.data_ptr(), kmax.data_ptr(),
            kmin.stride(0), kmin.stride(1), kmin.stride(2), scores.data_ptr(), P - 1, c["S"],
            c["S"] - 1, k, P - 1, kc.data_ptr(), vc.data_ptr(), kc.stride(0), kc.stride(1),
            kc.stride(2), kc.shape[2], None, 0, 0, pidx.data_ptr(), pidx.stride(0), pidx.stride(1),
            seqlens.data_ptr(), seqlens.stride(0), seqlens.stride(1), None, None, None,
            tau.data_ptr(), 2, out.data_ptr(), out.stride(0), out.stride(1), 1.5,
            qscale_for(1.5, D, dt), ps, B, H, Hkv, D, splits, max_tokens]
    code = {"fp32": 0, "fp16": 1, "bf16": 2}[c["dtype"]]
    stream = torch.cuda.current_stream(dev).cuda_stream
    if noalloc:
        _lib.call("ekv_topk_paged_entmax_decode_noalloc", *args, code, stream)
    else:
        nbytes = _lib.lib().ekv_decode_workspace_bytes(B, H, Hkv, D, splits, max_tokens)
        ws = torch.empty(int(nbytes), dtype=torch.uint8, device=dev)
        _lib.call("ekv_topk_paged_entmax_decode", *args, ws.data_ptr(), ws.numel(), code, stream)
    torch.cuda.synchronize()
    return out, pidx, tau, scores


def _same(c):
    ref = _run(c, noalloc=False)
    got = _run(c, noalloc=True)
    for name, r, g in zip(("out", "page table", "tau", "scores"), ref, got):
        assert torch.equal(r, g), name


def test_noalloc_matches_workspace_entry_point():
    print("CASE noalloc split B2 Hkv2 G4 400 pages k100, then B1 Hkv2 G4 150 pages k40",
          flush=True)
    _same(_case(2, 2, 4, 400, 100, "bf16", 1))
    _same(_case(1, 2, 4, 150, 40, "bf16", 2))
    print("CASE noalloc fused B8 Hkv16 G1 300 pages k64", flush=True)
    _same(_case(8, 16, 1, 300, 64, "fp16", 3))


def test_noalloc_rejects_a_step_beyond_the_scratch():
    from entmaxkv_amd import _lib
    print("CASE noalloc rejection", flush=True)
    B, H, Hkv, D, ps = 64, 64, 64, 128, 16
    max_tokens = 2048
    need = _lib.lib().ekv_decode_workspace_bytes(B, H, Hkv, D, 16, max_tokens)
    assert need > 16 << 20
    # every pointer null: were the size check to pass, the null-pointer check
    # behind it would still refuse the call, so nothing can launch
    args = [None, 0, 0, None, None, 0, 0, 0, None, 4096, 4096 * ps, 4096 * ps - 1, 127, 4095,
            None, None, 0, 0, 0, 4096 * ps, None, 0, 0, None, 0, 0, None, 0, 0, None, None,
            None, None, 2,
            None, 0, 0, 1.5, 0.0442, ps, B, H, Hkv, D, 16, max_tokens, 1,
            ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)]
    with pytest.raises(ValueError, match="static scratch"):
        _lib.call("ekv_topk_paged_entmax_decode_noalloc", *args)
