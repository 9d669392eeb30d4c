"""The reference-side ctypes stub printed in INTEGRATION.md runs as written.

The stub is the binding a maintainer of the reference would paste into
decode_flash_attention_redundant_var_len_paged.py (replacing the body of
flash_attention_decode_paged, :228-274) to call libakt_amd.so without this
package.  It declares its own argtypes, so these tests execute the document's
code block itself: on the CPU its declarations are checked against the header,
and on the GPU its paged decode is checked against the oracle and against the
package's own entry point (the same kernel, so bit-identical).
"""
import ctypes as C
import re
from pathlib import Path

import pytest

from attention_kernel_triton_amd import _native as N

ROOT = Path(__file__).resolve().parents[1]
DOC = ROOT / "INTEGRATION.md"
HEADER = ROOT / "include" / "akt_amd.h"


def _stub_source() -> str:
    text = DOC.read_text()
    blocks = re.findall(r"```python\n(.*?)```", text, flags=re.S)
    stubs = [b for b in blocks if "def flash_attention_decode_paged" in b]
    assert len(stubs) == 1, "INTEGRATION.md holds one paged-decode stub"
    src = stubs[0]
    assert '"/path/to/libakt_amd.so"' in src
    return src.replace('"/path/to/libakt_amd.so"', repr(str(N.library_path())))


def _load_stub() -> dict:
    ns: dict = {}
    exec(compile(_stub_source(), str(DOC), "exec"), ns)
    return ns


def _header_params(name: str) -> list[str]:
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    m = re.search(r"\b" + name + r"\s*\(([^)]*)\)\s*;", text)
    assert m, name
    return [a.strip() for a in m.group(1).split(",")]


def _kind(param: str):
    """ctypes type a header parameter binds to (pointers and arrays as pointers)."""
    if "*" in param or "[" in param:
        return "ptr"
    if param.startswith("int64_t"):
        return C.c_int64
    if param.startswith("size_t"):
        return C.c_size_t
    if param.startswith("float"):
        return C.c_float
    raise AssertionError(param)


def test_stub_argtypes_match_the_header():
    ns = _load_stub()
    lib = ns["_lib"]
    for fn in ("akt_decode_paged_fwd", "akt_decode_paged_workspace_size"):
        params = _header_params(fn)
        argtypes = getattr(lib, fn).argtypes
        assert len(argtypes) == len(params), fn
        for t, prm in zip(argtypes, params):
            k = _kind(prm)
            if k == "ptr":
                assert t is C.c_void_p or issubclass(t, C._Pointer), (fn, prm, t)
            else:
                assert t is k, (fn, prm, t)


@pytest.mark.gpu
def test_stub_paged_decode_matches_oracle_and_package(dev):
    import torch

    from attention_kernel_triton_amd import decode_flash_attention_redundant_var_len_paged as pg
    from attention_kernel_triton_amd import synthetic as syn
    from oracle import naive
    from tests.helpers import assert_close

    ns = _load_stub()
    p = syn.paged_config(B=6, Hq=16, Hkv=4, D=128, page=16, min_len=100, max_len=3000, seed=11)
    args = [t.to(dev) for t in (p.q, p.pool, p.indptr, p.indices, p.last_len)]
    o = ns["flash_attention_decode_paged"](*args)
    o2 = ns["flash_attention_decode_paged"](*args)  # the reused workspace is left zeroed
    torch.cuda.synchronize()
    ref, _ = naive.naive_paged_attention(p.q, p.pool, p.indptr, p.indices, p.last_len)
    assert_close(o.cpu(), ref, what="INTEGRATION.md stub")
    assert torch.equal(o, o2)
    assert torch.equal(o, pg.flash_attention_decode_paged(*args))
