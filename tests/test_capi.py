"""The C-ABI libraries load on a CPU-only host and export every function
their headers declare (include/allie_amd.h: liballie_amd.so,
include/allie_chess.h: liballie_chess.so); the ctypes tables bind exactly
those names.  No compute call is made on the GPU library (there is no GPU
here)."""
import ctypes
import glob
import os
import re

import pytest

from allie_amd import capi

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_signatures(header="allie_amd.h"):
    """name -> number of parameters, for every function the header declares."""
    sigs = {}
    for h in [os.path.join(ROOT, "include", header)]:
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


def test_every_header_is_covered():
    assert sorted(os.path.basename(h) for h in glob.glob(os.path.join(ROOT, "include", "*.h"))) == \
        ["allie_amd.h", "allie_chess.h"]


def test_chess_library_exports_every_declared_symbol():
    from allie_amd import rules

    if not os.path.exists(rules.LIB_PATH):
        pytest.skip("library not built (run __graft_entry__.build())")
    sigs = declared_signatures("allie_chess.h")
    assert len(sigs) >= 8
    lib = ctypes.CDLL(rules.LIB_PATH)
    for name in sigs:
        assert hasattr(lib, name), name
    L = rules.lib()
    for name, n_args in sigs.items():
        assert len(getattr(L, name).argtypes) == n_args, name


def test_library_missing_raises(monkeypatch, tmp_path):
    monkeypatch.setattr(capi, "_lib", None)
    monkeypatch.setattr(capi, "LIB_PATH", str(tmp_path / "nope.so"))
    with pytest.raises(capi.AllieError):
        capi.lib()


def test_gemm_split_factor_of_decode_shapes():
    """The K splits the forward picks for small-M projections (a host
    function; no GPU needed): unsplit at K = 1024 once M fills the CUs,
    more splits the fewer rows there are."""
    if not os.path.exists(capi.LIB_PATH):
        pytest.skip("library not built (run __graft_entry__.build())")
    f = capi.lib().allie_gemm_split_factor
    assert f(63, 1024, 4096) == 8    # decode-step MLP c_proj, 63 rows
    assert f(63, 3072, 1024) == 4    # decode-step QKV
    assert f(1024, 1024, 4096) == 4
    assert f(1450, 1024, 4096) == 2  # C4 step (about 1,450 rows)
    assert f(1450, 3072, 1024) == 1
    assert f(640, 1024, 1024) == 1   # attention c_proj of a C4 half-step (32+ tiles at K = 1024)
    assert f(256, 1024, 1024) == 4   # fewer tiles: still split
    for M in (1, 8, 64, 256, 1450, 53205):
        for N, K in ((3072, 1024), (1024, 1024), (4096, 1024), (1024, 4096)):
            s = f(M, N, K)
            assert s >= 1 and (K // 32) % s == 0
