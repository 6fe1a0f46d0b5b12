"""The C-ABI library loads and exports every symbol declared in include/*.h
(no compute: runs without a GPU)."""
import ctypes
import glob
import os
import re

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared():
    names = set()
    for h in glob.glob(os.path.join(ROOT, "include", "*.h")):
        text = open(h).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        names |= set(re.findall(r"\b(tallax_\w+)\s*\(", text))
    return sorted(names)


def test_header_symbols_exported():
    from tallax_amd import _lib
    lib = ctypes.CDLL(str(_lib._LIB_PATH))
    declared = _declared()
    assert len(declared) >= 6
    missing = [n for n in declared if not hasattr(lib, n)]
    assert not missing, missing
    # the Python binding knows every declared entry point
    assert set(declared) <= set(_lib.exported_symbols())


def test_error_path_without_gpu():
    from tallax_amd import _lib
    # invalid arguments are rejected on the host before any launch
    st = _lib.LIB.tallax_topk(None, 0, 4, 100, 8, None, None, None, 0, None)
    assert st == _lib.INVALID_ARGUMENT
    assert b"null" in _lib.LIB.tallax_last_error()
    st = _lib.LIB.tallax_topk(1, 0, 4, 100, 200, 1, 1, None, 0, None)
    assert st == _lib.UNSUPPORTED  # k > 128, like the reference's NotImplementedError
    # whole rows per workgroup need no workspace; segmented rows do
    assert _lib.LIB.tallax_topk_workspace_size(256, 128256, 128, 1) == 0
    assert _lib.LIB.tallax_topk_workspace_size(8, 200000, 64, 0) > 0


def test_sort_workspace_contract_without_gpu():
    from tallax_amd import _lib
    L = _lib.LIB
    # rows that fit one workgroup's LDS need no workspace
    assert L.tallax_sort_rows_workspace_size(256, 4096) == 0
    assert L.tallax_sort_rows_workspace_size(7, 16384) == 0
    # one merge pass: one record buffer; more: two (8 bytes per element each)
    assert L.tallax_sort_rows_workspace_size(3, 32768) == 3 * 32768 * 8
    assert L.tallax_sort_rows_workspace_size(1024, 201088) == 2 * 1024 * 201088 * 8
    # longer rows without (or with too little) workspace are refused before any launch
    st = L.tallax_sort_rows(1, 0, 2, 20000, 0, 0, None, 1, None, 0, None, 0, None, 0, None)
    assert st == _lib.WORKSPACE_TOO_SMALL
    assert b"workspace" in L.tallax_last_error()
    st = L.tallax_sort_rows_ws(1, 0, 2, 40000, 0, 0, None, 1, None, 0, None, 0, None, 0, 1, 100, None)
    assert st == _lib.WORKSPACE_TOO_SMALL
