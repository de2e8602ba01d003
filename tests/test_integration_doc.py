"""The ctypes binding that INTEGRATION.md shows a maintainer: its structs must
match the library's layout (the sizes luma_layout reports, and the field
offsets of luma_amd._lib's binding, which check_layout ties to the library)."""

import ctypes
import os
import re

import numpy as np

from luma_amd import _lib as L

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _doc_namespace():
    text = open(os.path.join(ROOT, "INTEGRATION.md")).read()
    blocks = re.findall(r"```python\n(.*?)```", text, flags=re.S)
    src = next(b for b in blocks if "class StepArgs" in b)
    # the definitions only: the dtypes and the ctypes struct (no library calls)
    keep = []
    for stmt in re.split(r"\n(?=\S)", src):
        if stmt.startswith(("TENSOR", "CHUNK", "GROUP", "class StepArgs")):
            keep.append(stmt)
    ns = {"np": np, "ctypes": ctypes}
    exec("\n".join(keep), ns)
    return ns


def test_doc_binding_matches_the_library_layout():
    ns = _doc_namespace()
    lib = L.load()
    out = (ctypes.c_int32 * 8)()
    lib.luma_layout(out)
    tensor_b, chunk_b, group_b, _, args_b = list(out)[:5]
    assert ns["TENSOR"].itemsize == tensor_b == L.TENSOR_DTYPE.itemsize
    assert ns["CHUNK"].itemsize == chunk_b
    assert ns["GROUP"].itemsize == group_b
    assert ctypes.sizeof(ns["StepArgs"]) == args_b
    doc = ns["StepArgs"]
    # same offsets as the package's binding (LumaScaling flattened in the doc)
    for name, _ in L.StepArgs._fields_:
        if name == "scaling":
            assert doc.grad_scale.offset == L.StepArgs.scaling.offset
            assert doc.found_inf.offset == L.StepArgs.scaling.offset + 8
        else:
            assert getattr(doc, name).offset == getattr(L.StepArgs, name).offset, name
    assert list(ns["TENSOR"].names) == list(L.TENSOR_DTYPE.names)
