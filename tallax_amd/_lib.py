"""ctypes binding of the C-ABI library `libtallax_hip.so` (declared in include/tallax_hip.h).

The product path always goes through this library.  If it is missing, the
import raises -- there is no CPU fallback.  Device buffers are torch tensors
(torch-ROCm is the allocator and stream provider only); every call is issued
on torch's current HIP stream of the tensor's device.
"""
from __future__ import annotations

import ctypes
import pathlib
import threading

import torch

_LIB_PATH = pathlib.Path(__file__).resolve().parent / "_build" / "libtallax_hip.so"

F32, BF16, I32 = 0, 1, 2
_DT = {torch.float32: F32, torch.bfloat16: BF16, torch.int32: I32}

# status codes (include/tallax_hip.h)
OK, INVALID_ARGUMENT, UNSUPPORTED, HIP_ERROR, WORKSPACE_TOO_SMALL = 0, 1, 2, 3, 4

_c_i64, _c_i32, _c_int, _c_sz, _c_p, _c_d = (
    ctypes.c_int64, ctypes.c_int32, ctypes.c_int, ctypes.c_size_t, ctypes.c_void_p, ctypes.c_double)

_SIGNATURES = {
    "tallax_last_error": ([], ctypes.c_char_p),
    "tallax_abi_version": ([], _c_int),
    "tallax_topk_workspace_size": ([_c_i64, _c_i64, _c_i64, _c_int], _c_sz),
    "tallax_topk": ([_c_p, _c_int, _c_i64, _c_i64, _c_i64, _c_p, _c_p, _c_p, _c_sz, _c_p], _c_int),
    "tallax_sample_workspace_size": ([_c_i64, _c_i64, _c_int], _c_sz),
    "tallax_fused_topk_topp_sample": (
        [_c_p, _c_int, _c_i64, _c_i64, _c_p, _c_p, _c_p, _c_p, _c_i64, _c_d, _c_p, _c_p, _c_sz, _c_p], _c_int),
    "tallax_fused_topk_topp_sample_noalloc": (
        [_c_p, _c_int, _c_i64, _c_i64, _c_p, _c_p, _c_p, _c_p, _c_i64, _c_d, _c_p, _c_p], _c_int),
    "tallax_sample_wide": ([_c_p, _c_int, _c_i64, _c_i64, _c_i64, _c_p, _c_p, _c_p, _c_p, _c_i64, _c_d, _c_p, _c_p,
                            _c_p, _c_p], _c_int),
    "tallax_shard_candidates_workspace_size": ([_c_i64, _c_i64, _c_int], _c_sz),
    "tallax_shard_candidates": ([_c_p, _c_int, _c_i64, _c_i64, _c_i64, _c_p, _c_p, _c_sz, _c_p], _c_int),
    "tallax_sample_from_candidates": ([_c_p, _c_i64, _c_int, _c_i64, _c_i64, _c_p, _c_p, _c_p, _c_p, _c_i64, _c_d,
                                       _c_p, _c_p], _c_int),
    "tallax_top_p_mask": ([_c_p, _c_i64, _c_i64, _c_p, _c_d, _c_p, _c_p], _c_int),
    "tallax_top_p_and_sample": (
        [_c_p, _c_int, _c_p, _c_i64, _c_i64, _c_p, _c_p, _c_p, _c_i64, _c_d, _c_i64, _c_p, _c_p], _c_int),
    "tallax_take_along_axis": ([_c_p, _c_int, _c_i64, _c_i64, _c_p, _c_i64, _c_i64, _c_int, _c_p, _c_p], _c_int),
    "tallax_cumsum": ([_c_p, _c_int, _c_i64, _c_i64, _c_int, _c_int, _c_p, _c_p], _c_int),
    "tallax_sort_rows": ([_c_p, _c_int, _c_i64, _c_i64, _c_int, _c_int, _c_p, _c_p, _c_p, _c_int, _c_p, _c_int,
                          _c_p, _c_int, _c_p], _c_int),
    "tallax_sort_rows_workspace_size": ([_c_i64, _c_i64], _c_sz),
    "tallax_gather_sort_key": ([_c_p, _c_int, _c_i64, _c_i64, _c_p, _c_p, _c_int, _c_p], _c_int),
    "tallax_sort_rows_ws": ([_c_p, _c_int, _c_i64, _c_i64, _c_int, _c_int, _c_p, _c_p, _c_p, _c_int, _c_p, _c_int,
                             _c_p, _c_int, _c_p, _c_sz, _c_p], _c_int),
    "tallax_topk_replace": ([_c_p, _c_int, _c_i64, _c_i64, _c_i64, _c_p, _c_d, _c_p, _c_p, _c_p, _c_sz, _c_p], _c_int),
    "tallax_top_dynamic_k_workspace_size": ([_c_i64, _c_int, _c_p, _c_int], _c_sz),
    "tallax_top_dynamic_k": ([_c_p, _c_int, _c_i64, _c_i64, _c_p, _c_int, _c_int, _c_int, _c_p, _c_int, _c_int,
                              _c_int, _c_d, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_sz, _c_p], _c_int),
    "tallax_softmax_topk_cumsum": ([_c_p, _c_i64, _c_i64, _c_int, ctypes.c_float, _c_p, _c_p, _c_p, _c_p, _c_p],
                                   _c_int),
    # test hooks (include/tallax_hip_testing.h)
    "tallax_testing_expf_logf": ([_c_p, _c_p, _c_p, _c_i64, _c_p], _c_int),
    "tallax_testing_gumbel": ([ctypes.c_uint32, ctypes.c_uint32, _c_p, _c_p, _c_p, _c_i64, _c_p], _c_int),
    "tallax_testing_lane_ops": ([_c_p, _c_p], _c_int),
    "tallax_testing_read_bytes": ([_c_p, _c_i64, _c_int, _c_p, _c_p], _c_int),
    "tallax_testing_lds_atomic_order": ([_c_p, _c_i64, _c_int, _c_p, _c_p], _c_int),
    "tallax_testing_select_plan": ([_c_i64, _c_i64, _c_int, _c_p], _c_int),
    "tallax_testing_top_dynamic_k_path": ([_c_p, _c_int, _c_i64, _c_i64, _c_p, _c_int, _c_int, _c_int, _c_p, _c_int,
                                           _c_int, _c_int, _c_d, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_sz, _c_p, _c_int],
                                          _c_int),
}


class TallaxError(RuntimeError):
    """Raised when the HIP library reports a failure."""


def _load() -> ctypes.CDLL:
    if not _LIB_PATH.exists():
        raise ImportError(
            f"tallax_amd HIP library not built: {_LIB_PATH} is missing. "
            "Run `python -c 'import __graft_entry__ as g; g.build()'` (hipcc, gfx950).")
    lib = ctypes.CDLL(str(_LIB_PATH))
    for name, (args, res) in _SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = res
    return lib


LIB = _load()


def exported_symbols() -> list[str]:
    return list(_SIGNATURES)


def check(status: int, what: str) -> None:
    if status == OK:
        return
    msg = LIB.tallax_last_error().decode(errors="replace")
    if status == UNSUPPORTED:
        raise NotImplementedError(f"{what}: {msg}")
    if status in (INVALID_ARGUMENT, WORKSPACE_TOO_SMALL):
        raise ValueError(f"{what}: {msg}")
    raise TallaxError(f"{what}: {msg} (status {status})")


def dtype_code(t: torch.Tensor) -> int:
    try:
        return _DT[t.dtype]
    except KeyError:
        raise NotImplementedError(f"dtype {t.dtype} is not supported (float32, bfloat16, int32)") from None


def stream_of(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


# ---------------------------------------------------------------------------
# Workspace: one byte buffer per device, grown on demand.  No kernel reads
# workspace contents it did not write in the same call, so the buffer never
# needs clearing.  Calls that overlap on one device (different streams) must
# pass their own workspace.  A buffer that growth supersedes is kept alive
# (never returned to the caching allocator), so work already enqueued on it,
# or a HIP graph captured with its address, never sees its memory reused.
# Growth is refused while the current stream is capturing: a capturing caller
# passes workspace= or warms the buffer up eagerly first.
# ---------------------------------------------------------------------------
_ws_lock = threading.Lock()
_ws: dict[int, torch.Tensor] = {}
_ws_retired: list[torch.Tensor] = []


def workspace(device: torch.device, nbytes: int) -> torch.Tensor:
    idx = device.index if device.index is not None else torch.cuda.current_device()
    with _ws_lock:
        buf = _ws.get(idx)
        if buf is None or buf.numel() < nbytes:
            if torch.cuda.is_current_stream_capturing():
                raise RuntimeError(
                    f"tallax_amd: the shared workspace of device {idx} must grow to {nbytes} bytes during "
                    "stream capture; pass workspace= or run the call once before capturing")
            if buf is not None:
                _ws_retired.append(buf)
            buf = torch.zeros(max(nbytes, 1 << 20), dtype=torch.uint8, device=torch.device("cuda", idx))
            _ws[idx] = buf
        return buf


def workspace_arg(workspace_t: torch.Tensor | None, device: torch.device, nbytes: int) -> torch.Tensor:
    """The caller's workspace (checked: a uint8 tensor on `device`, at least
    nbytes long) or the shared per-device one."""
    if workspace_t is None:
        return workspace(device, nbytes)
    if (not isinstance(workspace_t, torch.Tensor) or workspace_t.device != device
            or workspace_t.dtype != torch.uint8 or not workspace_t.is_contiguous()):
        raise ValueError("workspace must be a contiguous uint8 tensor on the operands' device")
    if workspace_t.numel() < nbytes:
        raise ValueError(f"workspace of {workspace_t.numel()} bytes is smaller than the {nbytes} required")
    return workspace_t


def require_cuda(*ts: torch.Tensor) -> None:
    for t in ts:
        if not isinstance(t, torch.Tensor) or not t.is_cuda:
            raise ValueError("tallax_amd operands must be torch tensors on a ROCm (cuda) device")
    devs = {t.device for t in ts}
    if len(devs) > 1:
        raise ValueError(f"operands on different devices: {devs}")


def select_plan(rows: int, cols: int, dtype: int, k: int = 128, sample: bool = True) -> dict:
    """Work split of the selection kernels for a [rows, cols] input (host only).
    A row is one whole-row workgroup (1024 threads, one segment), 2-4 equal
    whole-row parts (1024 threads, `segments` = parts) or 256-thread segments.
    Rows of several segments or parts finish in seg_merge64_pair_kernel (two
    lists) or seg_merge64_kernel for top-k with k <= 64 (no sampler), else in
    seg_merge_kernel."""
    out = (ctypes.c_int32 * 4)()
    check(LIB.tallax_testing_select_plan(rows, cols, dtype, out), "select_plan")
    nt, maxv, nseg, vps = list(out)
    dt = {F32: 0, BF16: 1}[dtype]
    merge = ("seg_merge64_pair_kernel" if nseg <= 2 else "seg_merge64_kernel") if (not sample and k <= 64) \
        else "seg_merge_kernel"
    if nt == 1024:
        # EDGE: rows (or parts) not a whole number of 16-byte vectors (a 16-byte aligned base assumed)
        edge = "true" if (cols // nseg * (4 if dtype == F32 else 2)) % 16 else "false"
        if nseg == 1:
            name = f"stream_select_kernel<{dt}, {maxv}, SAMPLE, {edge}>"
        else:
            name = f"stream_select_kernel<{dt}, {maxv}, false, {edge}> (parts) + {merge}"
    else:
        name = f"seg_select_kernel<{dt}, {maxv}, {nt}, SAMPLE>" + (f" + {merge}" if nseg > 1 else "")
    return {"threads": nt, "vectors_per_thread": maxv, "segments": nseg, "vectors_per_segment": vps,
            "kernel": name}
