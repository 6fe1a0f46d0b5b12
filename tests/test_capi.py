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
