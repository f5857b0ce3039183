"""ctypes binding of libentmaxkv_hip.so (the C ABI declared in include/entmaxkv.h).

The library is required: there is no CPU or PyTorch fallback.  ``lib()`` raises
``RuntimeError`` when the shared object is missing or fails to load, and every
wrapper raises when an entry point returns an error code.
"""

from __future__ import annotations

import ctypes
import os
import threading

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
# ENTMAXKV_AMD_LIB selects another build of the same library (e.g. a variant
# built for an experiment); the default is the in-tree build.
LIB_PATH = os.environ.get("ENTMAXKV_AMD_LIB", os.path.join(_HERE, "libentmaxkv_hip.so"))

P = ctypes.c_void_p
I = ctypes.c_int
I64 = ctypes.c_int64
F = ctypes.c_float

# name -> (restype, argtypes); mirrors include/entmaxkv.h
SIGNATURES = {
    "ekv_last_error": (ctypes.c_char_p, []),
    "ekv_abi_version": (I, []),
    "ekv_build_id": (ctypes.c_char_p, []),
    "ekv_page_stats": (I, [P, I64, I64, I64, P, P, P, P, I64, I64, I64, I, I, I, I, P, I, I, I, I,
                           P]),
    "ekv_append": (I, [P, P, I64, I64, P, P, I64, I64, I64, P, P, P, P, I64, I64, I64, I, I, I, I,
                       P, P, I64, I, I, I, P]),
    "ekv_page_criticality": (I, [P, I64, I64, P, P, I64, I64, I64, P, P, I, I, I, I, I, I, I, I, I,
                                 I, P, P, I64, I64, I, P]),
    "ekv_topk_pages": (I, [P, I, I, I, I, I, I, P, I64, I64, I, P]),
    "ekv_decode_workspace_bytes": (I64, [I, I, I, I, I, I]),
    "ekv_paged_entmax_decode": (I, [P, I64, I64, P, P, I64, I64, I64, I64, P, I64, I, P, I64, I64,
                                    I, P, I64, I64, P, P, P, P, I, I, P, I64, I64, F, F, I, I, I,
                                    I, I, I, I, P, I64, I, P]),
    "ekv_topk_paged_entmax_decode": (I, [P, I64, I64, P, P, I64, I64, I64, P, I, I, I, I, I, P, P,
                                         I64, I64, I64, I64, P, I64, I, P, I64, I64, P, I64, I64,
                                         P, P, P, P, I, P, I64, I64, F, F, I, I, I, I, I, I, I, P,
                                         I64, I, P]),
    "ekv_append_topk_paged_entmax_decode": (I, [P, P, I64, I64, P, P, I,
                                                P, I64, I64, P, P, I64, I64, I64, P, I, I, I, I,
                                                I, P, P, I64, I64, I64, I64, P, I64, I, P, I64,
                                                I64, P, I64, I64, P, P, P, P, I, P, I64, I64, F,
                                                F, I, I, I, I, I, I, I, P, I64, I, P]),
    "ekv_topk_paged_entmax_decode_noalloc": (I, [P, I64, I64, P, P, I64, I64, I64, P, I, I, I, I,
                                                 I, P, P, I64, I64, I64, I64, P, I64, I, P, I64,
                                                 I64, P, I64, I64, P, P, P, P, I, P, I64, I64, F,
                                                 F, I, I, I, I, I, I, I, I, P]),
    "ekv_gaussian_workspace_bytes": (I64, [I, I, I, I, I, I]),
    "ekv_gaussian_page_stats": (I, [P, I64, I64, P, P, I64, I64, I64, I, P, I, I, P, P, P, P, P, P,
                                    P, F, I, I, F, P, I, I, I, I, P, I64, I, P]),
    "ekv_gaussian_moments": (I, [P, I64, I64, P, P, I64, I64, I64, I, P, I, I, I, P, P, P, I, I, I,
                                 I, P, I64, I, P]),
    "ekv_gaussian_paged_entmax_decode": (I, [P, I64, P, P, I, I, P, P, P, P, P, I, I, I, F, I, F,
                                             F, F, F, F, P, I64, I64, P, P, P, I, P, F, F, P, P,
                                             I64, I64, P, P, I64, I64, I64, I64, P, I64, I, P, P,
                                             P, P, I, I, P, I64, I64, F, F, I, I, I, I, I, I, P,
                                             I64, I, P]),
    "ekv_tau_single_gaussian": (I, [P, P, P, I, I, F, I, F, P]),
    "ekv_tau_page_mixture": (I, [P, P, P, I, I, F, F, I, F, P, I, I, P]),
    "ekv_select_gaussian_pack": (I, [P, P, P, P, I, I, I, I, I, F, I, F, F, F, F, F, P, I64, I64,
                                     P, P, P, I, I, P, F, F, P, P, P]),
    "ekv_tau_clamp": (I, [P, P, P, P, I64, I64, I, P, I64, I64, P, P, I, I, I, I, F, F, F, P]),
    "ekv_cache_seqlens_from_counts": (I, [P, P, I, I, I, P]),
    "ekv_dense_decode_workspace_bytes": (I64, [I, I, I64]),
    "ekv_dense_entmax_decode": (I, [P, I64, I64, P, P, I64, I64, I64, I64, P, P, I64, I64, P, P, P,
                                    I, P, I64, I64, F, F, I, I, I, I, P, I64, I, P]),
    "ekv_entmax_rows_forward": (I, [P, I64, P, I64, I64, I, F, P, I, P]),
    "ekv_entmax_rows_backward": (I, [P, I64, P, I64, P, I64, I64, I, F, I, P]),
}

ABI_VERSION = 5

_lock = threading.Lock()
_lib = None


def lib():
    """Load the HIP library once; raise if it is absent or incompatible."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"entmaxkv_amd: {LIB_PATH} not found; build it with "
                "`python -m entmaxkv_amd.build` (hipcc, gfx950)")
        try:
            handle = ctypes.CDLL(LIB_PATH)
        except OSError as e:  # pragma: no cover - depends on the machine
            raise RuntimeError(f"entmaxkv_amd: cannot load {LIB_PATH}: {e}") from e
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        v = handle.ekv_abi_version()
        if v != ABI_VERSION:
            raise RuntimeError(f"entmaxkv_amd: library ABI {v}, expected {ABI_VERSION}; rebuild")
        _lib = handle
        return _lib


def build_id() -> str:
    """Source hash the loaded library was built from (ekv_build_id)."""
    return lib().ekv_build_id().decode()


def call(name: str, *args) -> None:
    rc = getattr(lib(), name)(*args)
    if rc != 0:
        msg = lib().ekv_last_error().decode(errors="replace")
        if rc == -1:
            raise ValueError(f"{name}: {msg}")
        raise RuntimeError(f"{name}: {msg}")


DTYPE_CODE = {torch.float32: 0, torch.float16: 1, torch.bfloat16: 2}


def dtype_code(dt: torch.dtype) -> int:
    try:
        return DTYPE_CODE[dt]
    except KeyError:
        raise TypeError(f"entmaxkv_amd: unsupported dtype {dt} (fp32, fp16, bf16)") from None


def ptr(t) -> int | None:
    return None if t is None else t.data_ptr()


def stream_ptr(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def require_gpu(*tensors) -> None:
    for t in tensors:
        if t is not None and not t.is_cuda:
            raise ValueError("entmaxkv_amd: tensors must live on the GPU (no CPU path)")
