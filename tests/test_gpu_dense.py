"""Dense utilities on the GPU vs the CPU oracle: row-wise entmax forward and
backward (and their autograd wrapper) and the dense (non-paged) decode."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import entmaxkv_oracle as O
from tests.gpu_helpers import ATOL, TORCH_DT, assert_out_close, randn, to_dev, to_np

pytestmark = pytest.mark.gpu

DTYPES = ["fp16", "bf16", "fp32"]


def _case(**kw):
    print("CASE", " ".join(f"{k}={v}" for k, v in kw.items()), flush=True)


# ---------------------------------------------------------------------------
# row-wise entmax
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("alpha", [1.5, 2.0, 1.25, 3.0])
# rows in registers (n <= 8192, 1..32 values per thread), in LDS (<= 16384)
# and re-read from memory (longer)
@pytest.mark.parametrize("n", [1, 7, 1000, 8192, 12000, 20000])
def test_entmax_rows_forward(dtype, alpha, n):
    from entmaxkv_amd.entmax import entmax_forward
    _case(test="entmax_rows_forward", dtype=dtype, alpha=alpha, n=n)
    rng = np.random.default_rng(n + int(alpha * 10))
    rows = 6
    x = randn(rng, (rows, n), dtype, 3.0)
    x[1, : min(n, 5)] = x[1, 0]  # ties
    xt = to_dev(x, dtype)
    tau = torch.empty(rows, dtype=torch.float32, device="cuda")
    y = entmax_forward(xt, alpha, tau_out=tau)
    torch.cuda.synchronize()
    ref_tau = np.array([O.entmax_tau_exact((alpha - 1.0) * r, alpha) for r in x])
    np.testing.assert_allclose(to_np(tau), ref_tau, atol=2e-6 * max(1.0, np.abs(ref_tau).max()))
    # the map at the kernel's own tau ((alpha - 1) x is exact in fp32 for these alphas)
    at_tau = np.stack([O.entmax_weights((alpha - 1.0) * r, t, alpha)
                       for r, t in zip(x, to_np(tau))])
    assert_out_close(to_np(y), at_tau, dtype, "y at tau")
    if alpha <= 2.0:
        # y is Lipschitz in tau here, so it also matches exact entmax; for
        # alpha > 2 ([d]_+^(1/(alpha-1)) has an unbounded slope at d = 0) a
        # tau within fp32 resolution moves y by up to sqrt(eps)
        assert_out_close(to_np(y), O.entmax_rows(x, alpha), dtype, "y")
    # exact tau: each fp32 row sums to 1 (alpha <= 2; for alpha > 2 the ulp of
    # tau alone moves the sum by up to ~sqrt(ulp) per support element near tau)
    if dtype == "fp32" and alpha <= 2.0:
        np.testing.assert_allclose(to_np(y).sum(-1), 1.0, atol=1e-5)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("alpha", [1.5, 2.0])
@pytest.mark.parametrize("n,rows", [(2048, 4200), (8192, 2100)])
def test_entmax_rows_forward_many_rows(dtype, alpha, n, rows):
    """More rows than resident workgroups: every workgroup of the register
    path solves several rows, loading the next row during the current one."""
    from entmaxkv_amd.entmax import entmax_forward
    _case(test="entmax_rows_forward_many_rows", dtype=dtype, alpha=alpha, n=n, rows=rows)
    rng = np.random.default_rng(rows + int(alpha * 10))
    x = randn(rng, (rows, n), dtype, 3.0)
    x[rows - 1, :5] = x[rows - 1, 0]  # ties in the last row
    x[rows // 2] = x[rows // 2, 0]    # an all-equal row: uniform output
    tau = torch.empty(rows, dtype=torch.float32, device="cuda")
    y = entmax_forward(to_dev(x, dtype), alpha, tau_out=tau)
    torch.cuda.synchronize()
    z = (alpha - 1.0) * x
    ref_tau = np.array([O.entmax_tau_exact(r, alpha) for r in z])
    np.testing.assert_allclose(to_np(tau), ref_tau, atol=2e-6 * max(1.0, np.abs(ref_tau).max()))
    assert_out_close(to_np(y), O.entmax_rows(x, alpha), dtype, "y")
    np.testing.assert_allclose(to_np(y)[rows // 2], 1.0 / n, atol=ATOL[dtype])


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("alpha", [1.5, 2.0, 1.25])
@pytest.mark.parametrize("n", [777, 4096, 10000])
def test_entmax_rows_backward_and_autograd(dtype, alpha, n):
    from entmaxkv_amd import entmax as E
    _case(test="entmax_rows_backward", dtype=dtype, alpha=alpha, n=n)
    rng = np.random.default_rng(7)
    shape = (2, 3, n)
    x = randn(rng, shape, dtype, 2.0)
    dy = randn(rng, shape, dtype)
    xt = to_dev(x, dtype).requires_grad_(True)
    y = E.triton_entmax(xt, alpha=alpha)
    y.backward(to_dev(dy, dtype))
    torch.cuda.synchronize()
    # the backward at the GPU's own y isolates the backward kernel
    ref = O.entmax_rows_backward(to_np(y), O.round_to(dy, dtype), alpha)
    assert_out_close(to_np(xt.grad), ref, dtype, "dx")
    # and the whole map against the oracle's forward + backward
    y_ref = O.entmax_rows(x, alpha)
    assert_out_close(to_np(y), y_ref, dtype, "y")
    if dtype == "fp32":
        np.testing.assert_allclose(to_np(xt.grad), O.entmax_rows_backward(y_ref, dy, alpha),
                                   atol=1e-4)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("n,rows", [(2048, 4200), (8192, 2100)])
def test_entmax_rows_backward_many_rows(dtype, n, rows):
    """More rows than resident workgroups in the backward's register path."""
    from entmaxkv_amd import entmax as E
    _case(test="entmax_rows_backward_many_rows", dtype=dtype, n=n, rows=rows)
    rng = np.random.default_rng(rows)
    x = randn(rng, (rows, n), dtype, 3.0)
    dy = randn(rng, (rows, n), dtype)
    xt = to_dev(x, dtype).requires_grad_(True)
    y = E.triton_entmax(xt, alpha=1.5)
    y.backward(to_dev(dy, dtype))
    torch.cuda.synchronize()
    ref = O.entmax_rows_backward(to_np(y), O.round_to(dy, dtype), 1.5)
    assert_out_close(to_np(xt.grad), ref, dtype, "dx")


def test_entmax_convenience_names_and_strides():
    from entmaxkv_amd.entmax import triton_entmax15, triton_sparsemax
    _case(test="entmax_convenience")
    rng = np.random.default_rng(8)
    x = randn(rng, (64, 300), "fp32")
    xt = to_dev(x, "fp32")
    y2 = triton_sparsemax(xt[:, :200])  # row stride 300, non-contiguous view
    y15 = triton_entmax15(xt.t().contiguous().t())  # column-major: copied to rows
    # rows starting 4 bytes past a 16-byte boundary: element-wise loads
    xw = randn(rng, (8, 2049), "fp16")
    yu = triton_entmax15(to_dev(xw, "fp16")[:, 1:])
    torch.cuda.synchronize()
    assert_out_close(to_np(y2), O.entmax_rows(x[:, :200], 2.0), "fp32", "sparsemax")
    assert_out_close(to_np(y15), O.entmax_rows(x, 1.5), "fp32", "entmax15")
    assert_out_close(to_np(yu), O.entmax_rows(xw[:, 1:], 1.5), "fp16", "unaligned")


# ---------------------------------------------------------------------------
# dense decode (kernels/adadecode.py:754-1016)
# ---------------------------------------------------------------------------

# "split": few heads; "head": batch * kv heads >= 128
DENSE_SHAPES = {"split": (2, 2), "head": (8, 16)}


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("alpha", [1.5, 2.0])
@pytest.mark.parametrize("G", [1, 4])
@pytest.mark.parametrize("alibi", [False, True])
@pytest.mark.parametrize("path", ["split", "head"])
def test_dense_decode_matches_oracle(dtype, alpha, G, alibi, path):
    from entmaxkv_amd.kernels import sparse_attention_decode_orchestrator
    _case(test="dense_decode", dtype=dtype, alpha=alpha, G=G, alibi=alibi, path=path)
    rng = np.random.default_rng(300 + G)
    B, Hkv = DENSE_SHAPES[path]
    H, S, D = Hkv * G, 1500, 128
    K = randn(rng, (B, Hkv, S, D), dtype)
    V = randn(rng, (B, Hkv, S, D), dtype)
    q = randn(rng, (B, H, 1, D), dtype)
    lens = rng.integers(1, S + 1, B)
    lens[0] = S
    slopes = rng.uniform(0.001, 0.05, H) if alibi else None
    pos = np.sort(rng.choice(3 * S, (B, Hkv, S)), axis=-1) if alibi else None
    # the query follows its last key (as in decoding), so the support's biases
    # stay small and fp32 scores keep their resolution
    q_sl = np.array([pos[b_, :, : lens[b_]].max() + 1 for b_ in range(B)]) if alibi else None
    out = torch.zeros(B, H, 1, D, dtype=TORCH_DT[dtype], device="cuda")
    taus = torch.empty(B, H, dtype=torch.float32, device="cuda")
    dev = lambda a: None if a is None else torch.tensor(a, device="cuda")
    sparse_attention_decode_orchestrator(
        to_dev(q, dtype), to_dev(K, dtype), to_dev(V, dtype), out,
        torch.tensor(lens, dtype=torch.int32, device="cuda"),
        dev(pos if pos is not None else np.zeros((B, Hkv, S), np.int32)),
        alibi_slopes=None if slopes is None else torch.tensor(slopes, dtype=torch.float32,
                                                              device="cuda"),
        alpha=alpha, niter=2, q_seqlens=dev(q_sl), taus_out=taus)
    torch.cuda.synchronize()
    ref, ref_tau = O.dense_entmax_decode(q[:, :, 0], K, V, lens, alpha, 2, dtype, slopes, pos,
                                         q_sl)
    assert_out_close(to_np(out)[:, :, 0], ref, dtype)
    np.testing.assert_allclose(to_np(taus), ref_tau, atol=1e-4)


@pytest.mark.parametrize("alibi", [False, True])
def test_dense_decode_long_cache_and_profile(alibi):
    """A cache longer than 2048 pages of 16 (the page grouping doubles; the
    scores go through the workspace of the split scoring launch), with and
    without explicit ALiBi positions, and the profile dict."""
    from entmaxkv_amd.kernels import sparse_attention_decode_orchestrator
    _case(test="dense_decode_long", alibi=alibi)
    rng = np.random.default_rng(9)
    dtype, B, H, S, D = "bf16", 1, 2, 40000, 64
    K = randn(rng, (B, H, S, D), dtype)
    V = randn(rng, (B, H, S, D), dtype)
    q = randn(rng, (B, H, 1, D), dtype, 3.0)
    lens = np.array([S - 5])
    slopes = np.array([0.01, 0.0005]) if alibi else None
    pos = np.sort(rng.choice(2 * S, (B, H, S), replace=False), axis=-1) if alibi else None
    q_sl = np.array([pos[0, :, : lens[0]].max() + 1]) if alibi else None
    dev = lambda a: None if a is None else torch.tensor(a, device="cuda")
    out = torch.zeros(B, H, 1, D, dtype=TORCH_DT[dtype], device="cuda")
    prof = {}
    for _ in range(2):
        sparse_attention_decode_orchestrator(
            to_dev(q, dtype), to_dev(K, dtype), to_dev(V, dtype), out,
            torch.tensor(lens, dtype=torch.int32, device="cuda"), dev(pos),
            alibi_slopes=None if slopes is None else torch.tensor(slopes, dtype=torch.float32,
                                                                  device="cuda"),
            alpha=1.5, niter=10, q_seqlens=dev(q_sl), profile=prof)
    torch.cuda.synchronize()
    ref, _ = O.dense_entmax_decode(q[:, :, 0], K, V, lens, 1.5, 10, dtype, slopes, pos, q_sl)
    assert_out_close(to_np(out)[:, :, 0], ref, dtype)
    assert prof["_count"] == 2 and prof["total"] > 0.0
    if alibi:
        return
    # converged (10 steps): exact entmax over all keys
    qs = O.scaled_query(q[:, :, 0], 1.5, dtype)
    for h in range(H):
        s = K[0, h, : lens[0]] @ qs[0, h]
        assert_out_close(to_np(out)[0, h, 0], O.entmax_exact(s, 1.5) @ V[0, h, : lens[0]], dtype,
                         "exact")


def test_dense_decode_rejects_bad_arguments():
    from entmaxkv_amd.kernels import sparse_attention_decode_orchestrator
    _case(test="dense_decode_errors")
    q = torch.zeros(1, 2, 1, 64, dtype=torch.float16, device="cuda")
    k = torch.zeros(1, 2, 32, 64, dtype=torch.float16, device="cuda")
    out = torch.zeros_like(q)
    lens = torch.tensor([32], dtype=torch.int32, device="cuda")
    with pytest.raises(ValueError):
        sparse_attention_decode_orchestrator(q, k, k, out, lens, None, bins=8)
    with pytest.raises(TypeError):
        sparse_attention_decode_orchestrator(q, k.float(), k.float(), out, lens, None)
