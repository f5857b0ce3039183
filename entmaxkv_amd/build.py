"""Builds libentmaxkv_hip.so (gfx950) from entmaxkv_amd/csrc/*.hip with hipcc.

Usage: python -m entmaxkv_amd.build   (or call build()).
Each source compiles in parallel to an object under entmaxkv_amd/_build/, then
one link writes the library next to this file so it travels with the tree.
decode_inst.hip compiles once per (storage dtype, GQA group) pair, so the
decode kernels of different pairs build in parallel.
"""

from __future__ import annotations

import concurrent.futures as cf
import glob
import hashlib
import os
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OBJ = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libentmaxkv_hip.so")
ARCH = "gfx950"

CFLAGS = [
    "-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}",
    # packed fp32 arithmetic is disabled for every kernel in this library
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-result",
]


# sources compiled once per variant: file -> [(object tag, -D flags)]
INSTANCES = {
    "decode_inst.hip": [(f".t{t}.g{g}", [f"-DEKV_INST_DTYPE={t}", f"-DEKV_INST_G={g}"])
                        for t in (0, 1, 2) for g in (1, 2, 4, 8)],
}


def hipcc() -> str:
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    cand = os.path.join(rocm, "bin", "hipcc")
    return cand if os.path.exists(cand) else "hipcc"


def _run(cmd):
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed ({res.returncode}): {' '.join(cmd)}\n"
                           f"{res.stdout}{res.stderr}")


def build_id(srcs) -> str:
    """First 16 hex digits of a SHA-256 over the sources, headers and flags."""
    h = hashlib.sha256()
    files = sorted(srcs) + sorted(glob.glob(os.path.join(CSRC, "*.h"))) + \
        sorted(glob.glob(os.path.join(HERE, "..", "include", "*.h")))
    for f in files:
        h.update(os.path.basename(f).encode() + b"\0")
        with open(f, "rb") as fh:
            h.update(fh.read())
    h.update(" ".join(CFLAGS).encode())
    h.update(repr(INSTANCES).encode())
    return h.hexdigest()[:16]


def build(verbose: bool = False) -> str:
    os.makedirs(OBJ, exist_ok=True)
    srcs = sorted(glob.glob(os.path.join(CSRC, "*.hip")))
    inc = ["-I", os.path.join(HERE, "..", "include")]
    bid = build_id(srcs)
    objs, cmds = [], []
    for src in srcs:
        base = os.path.basename(src)
        variants = INSTANCES.get(base, [("", [])])
        for tag, defs in variants:
            obj = os.path.join(OBJ, base + tag + ".o")
            objs.append(obj)
            cmds.append([hipcc(), *CFLAGS, *defs, f'-DEKV_BUILD_ID="{bid}"', *inc, "-c", src,
                         "-o", obj])
    workers = min(len(cmds), max(1, (os.cpu_count() or 2)))
    with cf.ThreadPoolExecutor(workers) as ex:
        for cmd, fut in zip(cmds, [ex.submit(_run, c) for c in cmds]):
            if verbose:
                print(" ".join(cmd), flush=True)
            fut.result()
    tmp = LIB + ".tmp"
    link = [hipcc(), "-shared", "-fPIC", f"--offload-arch={ARCH}", *objs, "-o", tmp]
    if verbose:
        print(" ".join(link), flush=True)
    _run(link)
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose=True))
