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


def test_work_split_without_gpu():
    """Every row that fits 1024 threads x 19 vectors goes to the whole-row
    kernel, at any row count; longer rows into 2-4 whole-row parts or into
    segments."""
    from tallax_amd import _lib
    for rows, cols, dt in [(1, 128256, _lib.BF16), (64, 128256, _lib.BF16), (8, 32768, _lib.F32),
                           (100, 65472, _lib.F32), (13, 167, _lib.F32), (256, 131058, _lib.BF16),
                           (1, 151936, _lib.BF16), (8, 65536, _lib.F32), (64, 77810, _lib.F32)]:
        p = _lib.select_plan(rows, cols, dt)
        assert p["threads"] == 1024 and p["segments"] == 1, (rows, cols, p)
        assert _lib.LIB.tallax_topk_workspace_size(rows, cols, 64, dt) == 0
    assert _lib.select_plan(1, 151936, _lib.BF16)["vectors_per_thread"] == 19
    assert _lib.select_plan(1, 128256, _lib.BF16)["vectors_per_thread"] == 16
    # rows that divide into 2-4 whole-row parts, at most 512 part workgroups
    for rows, cols, dt, np_ in [(1, 160000, _lib.BF16, 2), (8, 80000, _lib.F32, 2), (128, 151936, _lib.F32, 2),
                                (64, 201088, _lib.F32, 4), (128, 256000, _lib.F32, 4), (256, 256000, _lib.BF16, 2)]:
        p = _lib.select_plan(rows, cols, dt)
        assert p["threads"] == 1024 and p["segments"] == np_, (rows, cols, p)
    assert _lib.select_plan(128, 151936, _lib.F32, k=50, sample=False)["kernel"] == \
        "stream_select_kernel<0, 19, false, false> (parts) + seg_merge64_pair_kernel"
    # otherwise segments: too many part workgroups, or a row that does not divide
    for rows, cols, dt in [(256, 201088, _lib.F32), (512, 151936, _lib.F32), (4, 200003, _lib.F32),
                           (2048, 151936, _lib.F32)]:
        p = _lib.select_plan(rows, cols, dt)
        assert p["threads"] == 256 and p["segments"] > 1, (rows, cols, p)


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


def test_new_entry_points_validate_on_the_host():
    """Argument checks of the sharded sampler, top_p_mask and the sort-key
    gather run before any launch (no GPU needed)."""
    from tallax_amd import _lib
    L = _lib.LIB
    # shard candidates: a shard narrower than 128 columns, a negative offset
    assert L.tallax_shard_candidates(1, 1, 4, 100, 0, 1, None, 0, None) == _lib.UNSUPPORTED
    assert L.tallax_shard_candidates(1, 1, 4, 1000, -5, 1, None, 0, None) == _lib.INVALID_ARGUMENT
    assert L.tallax_shard_candidates(1, 1, 4, 1000, 0, None, None, 0, None) == _lib.INVALID_ARGUMENT
    assert L.tallax_shard_candidates_workspace_size(256, 16032, 1) == 0  # whole rows: no workspace
    # merge + sample: list counts outside [1, 32], a vocabulary below 128
    args = (1, 1, 1, 1, 0, -1e12, 1, None)  # top_k, top_p, temperature, key, dim0_offset, replace_val, out, stream
    assert L.tallax_sample_from_candidates(1, 33, 1, 4, 128256, *args) == _lib.UNSUPPORTED
    assert L.tallax_sample_from_candidates(1, 0, 1, 4, 128256, *args) == _lib.INVALID_ARGUMENT
    assert L.tallax_sample_from_candidates(1, 4, 1, 4, 100, *args) == _lib.INVALID_ARGUMENT
    # top_p_mask: more than 128 candidates per column
    assert L.tallax_top_p_mask(1, 129, 4, 1, -1e12, 1, None) == _lib.UNSUPPORTED
    assert L.tallax_top_p_mask(1, 0, 4, 1, -1e12, 1, None) == _lib.INVALID_ARGUMENT
    # sort-key gather: an output dtype a key cannot decode to
    assert L.tallax_gather_sort_key(1, _lib.F32, 2, 10, 1, 1, _lib.BF16, None) == _lib.INVALID_ARGUMENT
    assert L.tallax_gather_sort_key(1, 7, 2, 10, 1, 1, _lib.F32, None) == _lib.UNSUPPORTED


def test_wide_sampler_validates_on_the_host():
    """tallax_sample_wide rejects widths outside [1, 1024] or above the
    vocabulary, and calls with nothing to write, before any launch."""
    from tallax_amd import _lib
    L = _lib.LIB
    par = (1, 1, 1, 1, 0, -1e12)  # top_k, top_p, temperature, key, dim0_offset, replace_val
    assert L.tallax_sample_wide(1, 1, 4, 128256, 1025, *par, 1, None, None, None) == _lib.UNSUPPORTED
    assert L.tallax_sample_wide(1, 1, 4, 128256, 0, *par, 1, None, None, None) == _lib.INVALID_ARGUMENT
    assert L.tallax_sample_wide(1, 1, 4, 500, 501, *par, 1, None, None, None) == _lib.INVALID_ARGUMENT
    assert L.tallax_sample_wide(1, 1, 4, 128256, 1024, *par, None, None, None, None) == _lib.INVALID_ARGUMENT
    assert L.tallax_sample_wide(1, 2, 4, 128256, 1024, *par, 1, None, None, None) == _lib.UNSUPPORTED
    assert L.tallax_sample_wide(1, 1, 4, 128256, 1024, None, 1, 1, 1, 0, -1e12, 1, None, None, None) \
        == _lib.INVALID_ARGUMENT
    assert L.tallax_sample_wide(1, 1, 0, 128256, 1024, None, None, None, None, 0, -1e12, None, 1, None, None) \
        == _lib.OK



def test_noalloc_sampler_limit_without_gpu():
    """The no-allocation sampler refuses, on the host and before any device
    call, inputs whose candidate lists exceed its 16 MiB scratch."""
    from tallax_amd import _lib
    L = _lib.LIB
    rows, vocab = 4096, 151936
    assert L.tallax_sample_workspace_size(rows, vocab, _lib.F32) > 16 << 20
    st = L.tallax_fused_topk_topp_sample_noalloc(1, _lib.F32, rows, vocab, 1, 1, 1, 1, 0, -1e12, 1, None)
    assert st == _lib.UNSUPPORTED
    assert b"scratch" in L.tallax_last_error()


def test_top_dynamic_k_path_hook_rejects_unknown_paths():
    from tallax_amd import _lib
    sched = (ctypes.c_int32 * 2)(3, 6)
    st = _lib.LIB.tallax_testing_top_dynamic_k_path(1, 0, 8, 100, 1, 4, 8, 128, sched, 2, 0, 0, 0.0, 1, 1, 1, 1, 1,
                                                    1, 1 << 20, None, 7)
    assert st == _lib.INVALID_ARGUMENT and b"path" in _lib.LIB.tallax_last_error()
