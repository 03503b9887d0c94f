"""The C-ABI library loads on a CPU-only host and exports every function
that include/*.h declares; the ctypes table binds exactly those names.
No compute call is made (there is no GPU here)."""
import ctypes
import glob
import os
import re

import pytest

from allie_amd import capi

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_signatures():
    """name -> number of parameters, for every function in include/*.h."""
    sigs = {}
    for h in glob.glob(os.path.join(ROOT, "include", "*.h")):
        src = open(h).read()
        src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
        for m in re.finditer(r"^\s*(?:const\s+)?[a-z_0-9]+\s*\*?\s*(allie_[a-z_0-9]+)\s*\(([^)]*)\)\s*;",
                             src, flags=re.M):
            params = " ".join(m.group(2).split())
            sigs[m.group(1)] = 0 if params in ("", "void") else params.count(",") + 1
    return sigs


def declared_functions():
    return sorted(declared_signatures())


def test_ctypes_signatures_match_header():
    sigs = declared_signatures()
    for name, res, args in capi._SIGS:
        assert name in sigs, name
        assert len(args) == sigs[name], (name, len(args), sigs[name])


def test_library_exports_every_declared_symbol():
    if not os.path.exists(capi.LIB_PATH):
        pytest.skip("library not built (run __graft_entry__.build())")
    lib = ctypes.CDLL(capi.LIB_PATH)
    decl = declared_functions()
    assert len(decl) >= 10
    for name in decl:
        assert hasattr(lib, name), name
    assert sorted(capi.EXPORTED) == decl
    # binding works and the pure-host entry points answer
    L = capi.lib()
    assert L.allie_abi_version() >= 1
    assert L.allie_prefill_workspace_bytes(None, 1, 1) == 0
    assert L.allie_model_create(None, None) == -1
    assert b"NULL" in L.allie_last_error()


def test_library_missing_raises(monkeypatch, tmp_path):
    monkeypatch.setattr(capi, "_lib", None)
    monkeypatch.setattr(capi, "LIB_PATH", str(tmp_path / "nope.so"))
    with pytest.raises(capi.AllieError):
        capi.lib()
