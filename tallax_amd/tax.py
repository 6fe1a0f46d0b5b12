"""lax-like API (mirror of tallax/tax.py: sort, top_k, top_dynamic_k, cumsum).

Operands are torch tensors on a ROCm device; every op runs a hand-written
gfx950 HIP kernel through the C ABI in include/tallax_hip.h.  TPU-only
keyword arguments of the reference (`interpret`, `block_token`,
`bins_topm_unroll`, `num_vmem_substages`) are accepted and ignored.
"""
from __future__ import annotations

import numbers

import torch

from . import _lib

NUM_LANES = 128  # tallax/_src/utils.py:13


def _canonical_2d(x: torch.Tensor) -> None:
    # utils.py:172-181: only 2D operands
    if x.ndim != 2:
        raise ValueError("Only 2D inputs supported")


def top_k(logits: torch.Tensor, k: int, block_token: int = 8, num_bins: int = NUM_LANES,
          bins_topm_unroll: int = 32, bins_topm_schedule=None, interpret: bool = False,
          *, workspace: torch.Tensor | None = None):
    """Exact top-k along the last axis: (values [R, k] descending, int32 indices [R, k]).

    Reference: top_k (tallax/_src/top_k.py:516-567).  Ties are broken to the
    lowest index.  k > 128 raises NotImplementedError as in the reference
    (top_k.py:438-439).  float32, bfloat16 and int32 logits (the reference is
    dtype-generic, utils.py:48-56): slots only the dtype's min (or NaN, -inf)
    could fill hold the dtype's min.
    """
    del block_token, num_bins, bins_topm_unroll, bins_topm_schedule, interpret
    _lib.require_cuda(logits)
    _canonical_2d(logits)
    k = int(k)
    if k > NUM_LANES:
        raise NotImplementedError(f"k={k} > {NUM_LANES}")
    rows, cols = logits.shape
    if k < 1 or k > cols:
        raise ValueError(f"k={k} must be in [1, {cols}]")
    x = logits.contiguous()
    dt = _lib.dtype_code(x)
    vals = torch.empty((rows, k), dtype=x.dtype, device=x.device)
    idx = torch.empty((rows, k), dtype=torch.int32, device=x.device)
    need = _lib.LIB.tallax_topk_workspace_size(rows, cols, k, dt)
    ws = _lib.workspace_arg(workspace, x.device, need)
    _lib.check(_lib.LIB.tallax_topk(
        x.data_ptr(), dt, rows, cols, k, vals.data_ptr(), idx.data_ptr(),
        ws.data_ptr() if need else None, ws.numel() if need else 0, _lib.stream_of(x)), "top_k")
    return vals, idx


def _k_rows(k, rows: int, device) -> torch.Tensor:
    if isinstance(k, numbers.Integral):
        # filled on the device: no host-to-device copy, so the call can be graph-captured
        return torch.full((rows,), int(k), dtype=torch.int32, device=device)
    t = k if isinstance(k, torch.Tensor) else torch.tensor(k, dtype=torch.int32)
    t = t.to(device=device, dtype=torch.int32)
    if t.ndim == 0:
        t = t.expand(rows)
    if tuple(t.shape) != (rows,):
        raise ValueError(f"k has shape {tuple(t.shape)}, expected () or ({rows},)")
    return t.contiguous()


def top_dynamic_k(logits: torch.Tensor, k, max_k: int, block_token: int = 8, num_bins: int = NUM_LANES,
                  bins_topm_unroll: int = 32, bins_topm_schedule=None, guarantee_convergence: bool = False,
                  replace_val=None, interpret: bool = False, *, workspace: torch.Tensor | None = None):
    """Per-row top-k (k <= max_k <= 128) by binned top-m supersets.

    Reference: top_dynamic_k (tallax/_src/top_k.py:385-514).
      * guarantee_convergence=False: the binned algorithm, returning
        (vals [R, max_k], idxs [R, max_k] int32, valid (bool scalar tensor),
        depths [R] int32, cutoff_vals [R] float32 -- int32 for int32 logits,
        the reference's to_32bit_dtype, top_k.py:465).  Bins are columns mod
        num_bins; the schedule (auto from the convergence theory if None)
        decides depths/cutoffs; the result is the top-128 of the first
        depth_upper ranks of every bin, ordered by value then lowest index.
      * guarantee_convergence=True: (vals, idxs) of the same algorithm,
        where a block of rows that has not converged after the last step
        (when that step's depth m is not max_k) first goes through the
        bin-packing merge (_merge_unconverged_bins_top_k, top_k.py:108-200):
        the 2^ceil(log2(ceil(max_k / (m - 1)))) bins with the most entries
        above the last pivot are packed whole and their top-128 replaces rank
        0 of bins 0..127.  Like the reference, no max_k step is added to the
        schedule; this needs m >= 2 and num_bins % 128 == 0 (ValueError /
        NotImplementedError otherwise).  For the exact answer use tax.top_k.
    Positions >= k[row] hold replace_val (in the logits dtype; int32 logits
    take it converted toward zero, saturated at the int32 range) when given.
    Raises ValueError if rows % block_token != 0 and NotImplementedError for
    max_k > 128, like the reference.  `workspace` (keyword only): a uint8
    device tensor of at least the entry point's workspace size, used instead
    of the shared per-device buffer (for callers that capture graphs or run
    calls concurrently).
    """
    return _top_dynamic_k(logits, k, max_k, block_token, num_bins, bins_topm_unroll, bins_topm_schedule,
                          guarantee_convergence, replace_val, interpret, workspace, None)


def _top_dynamic_k(logits, k, max_k, block_token, num_bins, bins_topm_unroll, bins_topm_schedule,
                   guarantee_convergence, replace_val, interpret, workspace, testing_path):
    """top_dynamic_k; testing_path 0/1 routes the binned form through the
    testing entry point that forces the candidate (0) or the scan (1) path."""
    del bins_topm_unroll, interpret
    from . import schedule as sch
    _lib.require_cuda(logits)
    _canonical_2d(logits)
    rows, cols = logits.shape
    if rows % block_token != 0:
        raise ValueError("num_tokens must be divisible by block_token")
    max_k = int(max_k)
    if max_k > NUM_LANES:
        raise NotImplementedError(f"max_k={max_k} > {NUM_LANES}")
    x = logits.contiguous()
    dt = _lib.dtype_code(x)
    kr = _k_rows(k, rows, x.device)
    dev = x.device
    stream = _lib.stream_of(x)
    vals = torch.empty((rows, max_k), dtype=x.dtype, device=dev)
    idx = torch.empty((rows, max_k), dtype=torch.int32, device=dev)
    steps = sch.topm_schedule(max_k, num_bins, block_token, bins_topm_schedule)
    if guarantee_convergence and steps[-1] != max_k:
        if steps[-1] < 2:
            raise ValueError(f"guarantee_convergence needs a last schedule depth >= 2 (or = max_k), got {steps[-1]}")
        if num_bins % NUM_LANES:
            raise NotImplementedError(f"guarantee_convergence needs num_bins % {NUM_LANES} == 0, got {num_bins}")
    import ctypes
    arr = (ctypes.c_int32 * len(steps))(*steps)
    need = _lib.LIB.tallax_top_dynamic_k_workspace_size(rows, num_bins, arr, len(steps))
    ws = _lib.workspace_arg(workspace, dev, max(need, 1))
    valid = torch.empty(1, dtype=torch.int32, device=dev)
    depths = torch.empty(rows, dtype=torch.int32, device=dev)
    cutoff = torch.empty(rows, dtype=torch.int32 if dt == _lib.I32 else torch.float32, device=dev)
    args = (x.data_ptr(), dt, rows, cols, kr.data_ptr(), max_k, block_token, num_bins, arr, len(steps),
            int(bool(guarantee_convergence)), int(replace_val is not None), float(replace_val) if replace_val is not None else 0.0, vals.data_ptr(),
            idx.data_ptr(), valid.data_ptr(), depths.data_ptr(), cutoff.data_ptr(), ws.data_ptr(), ws.numel(),
            stream)
    if testing_path is None:
        _lib.check(_lib.LIB.tallax_top_dynamic_k(*args), "top_dynamic_k")
    else:
        _lib.check(_lib.LIB.tallax_testing_top_dynamic_k_path(*args, int(testing_path)), "top_dynamic_k")
    if guarantee_convergence:
        return vals, idx
    return vals, idx, valid.reshape(()).bool(), depths, cutoff


_SORT_DTYPES = (torch.float32, torch.bfloat16, torch.int32)


def sort(operand, num_keys: int, is_stable: bool = False, return_argsort: bool = False,
         descending: bool = False, num_vmem_substages=None, block_token=None, interpret: bool = False) -> tuple:
    """Row-wise lexicographic sort of one or more 2D operands by the first
    `num_keys` of them.

    Reference: sort (tallax/_src/sort.py:768-929).  Mirrors its host logic:
      * integer operands with a non-power-of-two row force a stable sort
        (sort.py:798-802);
      * stable / argsort insert the column index as a tie-breaking key;
        descending + stable keeps ties in ascending index order
        (sort.py:804-813, 925-926);
      * a bfloat16 key sorted together with only the index (rows <= 65536)
        takes the packed path and comes back as bfloat16 (NaN -> 0x7FFF,
        sort.py:823-831, utils.py:205-227); otherwise float keys come back
        standardised and decoded (-0 -> +0, NaN -> 0x7FFFFFFE), bfloat16 keys
        as float32 (utils.py:139-147 promotes them);
      * non-key operands are permuted unchanged; with return_argsort the
        int32 indices are appended last.
    Non-stable ties are ordered by ascending index (the reference leaves that
    order to its network).  Keys: float32, bfloat16, int32, any number of
    them; rows of any length below 2^31.  Rows longer than 16384 elements (the
    reference's HBM substage route, sort.py:574-758) are sorted in chunks and
    merged through a device workspace of 8 or 16 bytes per element.
    `num_vmem_substages`, `block_token` and `interpret` are TPU tuning knobs,
    accepted and ignored.
    """
    del num_vmem_substages, block_token, interpret
    operands = list(operand) if isinstance(operand, (list, tuple)) else [operand]
    if not operands:
        raise ValueError("sort needs at least one operand")
    _lib.require_cuda(*operands)
    shapes = {tuple(x.shape) for x in operands}
    if len(shapes) != 1:
        raise ValueError(f"Inputs must all have the same shape, but found shapes={[tuple(x.shape) for x in operands]}")
    shape = shapes.pop()
    if len(shape) != 2:
        raise ValueError("Only 2D inputs supported")
    num_keys = int(num_keys)
    if not 1 <= num_keys <= len(operands):
        raise ValueError(f"num_keys={num_keys} must be in [1, {len(operands)}]")
    for x in operands:
        if x.dtype not in _SORT_DTYPES:
            raise NotImplementedError(f"sort operand dtype {x.dtype}")
    rows, cols = shape
    if cols & (cols - 1) and any(not x.dtype.is_floating_point for x in operands):
        is_stable = True
    use_indices = return_argsort or is_stable
    packed = (operands[0].dtype == torch.bfloat16 and len(operands) + int(use_indices) == 2 and use_indices
              and cols <= 2 ** 16)
    ties_desc = packed and descending and not is_stable
    ops = [x.contiguous() for x in operands]
    dev = ops[0].device
    stream = _lib.stream_of(ops[0])

    def key_out_dtype(x):
        if x.dtype == torch.bfloat16:
            return torch.bfloat16 if packed else torch.float32
        return x.dtype

    perm = torch.empty(shape, dtype=torch.int32, device=dev)
    outs = [None] * len(ops)
    k0 = ops[0]
    out0 = torch.empty(shape, dtype=key_out_dtype(k0), device=dev)
    # rows longer than 16384: a per-call workspace (the caching allocator recycles it)
    nws = int(_lib.LIB.tallax_sort_rows_workspace_size(rows, cols))
    ws = torch.empty(nws, dtype=torch.uint8, device=dev) if nws else None
    ws_ptr = ws.data_ptr() if ws is not None else None
    if num_keys == 1:
        _lib.check(_lib.LIB.tallax_sort_rows_ws(
            k0.data_ptr(), _lib.dtype_code(k0), rows, cols, int(bool(descending)), int(ties_desc), None,
            perm.data_ptr(), out0.data_ptr(), _lib.dtype_code(out0), None, 0, None, 0, ws_ptr, nws, stream), "sort")
    else:
        # stable LSD passes, last key first; each pass sorts key[perm] with
        # position ties and composes, so the final permutation orders the rows
        # lexicographically by all keys, ties by ascending index
        prev = None
        for i in range(num_keys - 1, 0, -1):
            ki = ops[i]
            pi = torch.empty(shape, dtype=torch.int32, device=dev)
            _lib.check(_lib.LIB.tallax_sort_rows_ws(
                ki.data_ptr(), _lib.dtype_code(ki), rows, cols, int(bool(descending)), 0,
                prev.data_ptr() if prev is not None else None, pi.data_ptr(), None, 0, None, 0, None, 0, ws_ptr, nws,
                stream), "sort")
            prev = pi
        k1 = ops[1]
        out1 = torch.empty(shape, dtype=key_out_dtype(k1), device=dev)
        _lib.check(_lib.LIB.tallax_sort_rows_ws(
            k0.data_ptr(), _lib.dtype_code(k0), rows, cols, int(bool(descending)), 0, prev.data_ptr(),
            perm.data_ptr(), out0.data_ptr(), _lib.dtype_code(out0), k1.data_ptr(), _lib.dtype_code(k1),
            out1.data_ptr(), _lib.dtype_code(out1), ws_ptr, nws, stream), "sort")
        outs[1] = out1
        for i in range(2, num_keys):  # further keys: gathered by the final permutation, decoded like keys
            ki = ops[i]
            oi = torch.empty(shape, dtype=key_out_dtype(ki), device=dev)
            _lib.check(_lib.LIB.tallax_gather_sort_key(ki.data_ptr(), _lib.dtype_code(ki), rows, cols,
                                                       perm.data_ptr(), oi.data_ptr(), _lib.dtype_code(oi), stream),
                       "sort")
            outs[i] = oi
    outs[0] = out0
    for i in range(num_keys, len(ops)):
        x = ops[i]
        o = torch.empty(shape, dtype=x.dtype, device=dev)
        _lib.check(_lib.LIB.tallax_take_along_axis(x.data_ptr(), _lib.dtype_code(x), rows, cols, perm.data_ptr(),
                                                   rows, cols, 1, o.data_ptr(), stream), "sort payload")
        outs[i] = o
    if return_argsort:
        outs.append(perm)
    return tuple(outs)


def _axis2(axis: int) -> int:
    axis = int(axis)
    if axis < 0:
        axis += 2
    if axis not in (0, 1):
        raise ValueError(f"axis {axis} out of range for a 2D operand")
    return axis


def cumsum(arr: torch.Tensor, axis: int, reverse: bool = False, interpret: bool = False) -> torch.Tensor:
    """Inclusive cumulative sum along `axis` (0 or 1) in the reference's order.

    Reference: cumsum (tallax/_src/cumsum.py:75-101): Hillis-Steele scans
    inside (8, 128) tiles plus a sequential carry of tile totals; dtype is
    preserved (float32 and int32 here; cast bfloat16 to float32 first, as the
    reference's docstring advises).  Negative axes are normalised (the
    reference's `1 - axis` batch axis only works for 0 and 1).
    """
    del interpret
    _lib.require_cuda(arr)
    _canonical_2d(arr)
    axis = _axis2(axis)
    x = arr.contiguous()
    dt = _lib.dtype_code(x)
    if dt == _lib.BF16:
        raise NotImplementedError("cumsum on bfloat16: cast to float32 first")
    out = torch.empty_like(x)
    rows, cols = x.shape
    _lib.check(_lib.LIB.tallax_cumsum(x.data_ptr(), dt, rows, cols, axis, int(bool(reverse)), out.data_ptr(),
                                      _lib.stream_of(x)), "cumsum")
    return out


__all__ = ["sort", "top_k", "top_dynamic_k", "cumsum"]
