"""Loads the reference-side ctypes binding that the integration guide gives, as a module.

The block is the text a maintainer would paste into the reference package as
``entmaxkv/kernels/_amd.py``; running it from the document keeps the document
and the library's ABI from drifting apart.
"""

import os
import re
import types

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
DOC = os.path.join(ROOT, "INTEGRATION.md")
MARK = "# entmaxkv/kernels/_amd.py"


def snippet_source() -> str:
    txt = open(DOC).read()
    blocks = re.findall(r"```python\n(.*?)```", txt, flags=re.S)
    found = [b for b in blocks if b.startswith(MARK)]
    assert len(found) == 1, "the integration guide must hold exactly one reference-side binding block"
    return found[0]


def load_snippet(lib_path: str) -> types.ModuleType:
    old = os.environ.get("ENTMAXKV_AMD_LIB")
    os.environ["ENTMAXKV_AMD_LIB"] = lib_path
    try:
        mod = types.ModuleType("entmaxkv_reference_amd_binding")
        exec(compile(snippet_source(), DOC, "exec"), mod.__dict__)
    finally:
        if old is None:
            del os.environ["ENTMAXKV_AMD_LIB"]
        else:
            os.environ["ENTMAXKV_AMD_LIB"] = old
    return mod
