"""CPU checks of the C ABI: the built library loads and exports exactly what
include/entmaxkv.h declares, with the argument counts the ctypes binding uses.
No compute entry point is called (there is no GPU here)."""

import os
import re
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "entmaxkv.h")


def _declared():
    txt = open(HEADER).read()
    txt = re.sub(r"/\*.*?\*/", "", txt, flags=re.S)
    decls = {}
    for m in re.finditer(r"\b(?:const\s+char\s*\*|int64_t|int)\s+(ekv_\w+)\s*\(([^;]*?)\)\s*;", txt, re.S):
        args = m.group(2).strip()
        n = 0 if args in ("", "void") else len([a for a in args.split(",") if a.strip()])
        decls[m.group(1)] = n
    return decls


def test_header_parses():
    d = _declared()
    assert "ekv_paged_entmax_decode" in d and len(d) >= 15


def test_library_exports_every_declared_symbol():
    from entmaxkv_amd import _lib
    lib = _lib.lib()  # loads, checks the ABI version
    decl = _declared()
    for name, nargs in decl.items():
        assert hasattr(lib, name), name
        assert name in _lib.SIGNATURES, f"{name} missing from the ctypes table"
        assert len(_lib.SIGNATURES[name][1]) == nargs, f"{name}: {nargs} args in the header"
    out = subprocess.run(["nm", "-D", "--defined-only", _lib.LIB_PATH], capture_output=True,
                         text=True).stdout
    exported = set(re.findall(r" T (ekv_\w+)", out))
    assert exported == set(decl), exported ^ set(decl)


def test_product_path_fails_loudly_without_gpu_tensors():
    import torch
    from entmaxkv_amd import PagedKVCache
    c = PagedKVCache()
    with pytest.raises(ValueError):
        c.initialize(torch.zeros(1, 1, 16, 64), torch.zeros(1, 1, 16, 64))


def test_missing_library_raises(monkeypatch, tmp_path):
    from entmaxkv_amd import _lib
    monkeypatch.setattr(_lib, "_lib", None)
    monkeypatch.setattr(_lib, "LIB_PATH", str(tmp_path / "nope.so"))
    with pytest.raises(RuntimeError):
        _lib.lib()


def test_integration_snippet_matches_the_abi():
    """The integration guide's reference-side ctypes block declares, and passes,
    exactly the parameters of ekv_page_criticality."""
    import ast
    import ctypes

    from entmaxkv_amd import _lib
    from integration_snippet import load_snippet, snippet_source

    mod = load_snippet(_lib.LIB_PATH)
    argtypes = mod._lib.ekv_page_criticality.argtypes
    want = _lib.SIGNATURES["ekv_page_criticality"][1]
    assert len(argtypes) == _declared()["ekv_page_criticality"] == len(want)
    for i, (a, b) in enumerate(zip(argtypes, want)):
        assert a is b, (i, a, b)
    calls = [n for n in ast.walk(ast.parse(snippet_source()))
             if isinstance(n, ast.Call) and getattr(n.func, "attr", "") == "ekv_page_criticality"]
    assert len(calls) == 1 and len(calls[0].args) == len(argtypes)
