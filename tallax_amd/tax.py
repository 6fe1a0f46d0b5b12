"""lax-like API (mirror of tallax/tax.py: sort, top_k, top_dynamic_k, cumsum).

Operands are torch tensors on a ROCm device; every op runs a hand-written
gfx950 HIP kernel through the C ABI in include/tallax_hip.h.  TPU-only
keyword arguments of the reference (`interpret`, `block_token`,
`bins_topm_unroll`, `num_vmem_substages`) are accepted and ignored.
"""
from __future__ import annotations

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
    (top_k.py:438-439).
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
    if dt == _lib.I32:
        raise NotImplementedError("top_k on int32 logits is not supported")
    vals = torch.empty((rows, k), dtype=x.dtype, device=x.device)
    idx = torch.empty((rows, k), dtype=torch.int32, device=x.device)
    need = _lib.LIB.tallax_topk_workspace_size(rows, cols, k, dt)
    ws = workspace if workspace is not None else _lib.workspace(x.device, need)
    _lib.check(_lib.LIB.tallax_topk(
        x.data_ptr(), dt, rows, cols, k, vals.data_ptr(), idx.data_ptr(),
        ws.data_ptr() if need else None, ws.numel() if need else 0, _lib.stream_of(x)), "top_k")
    return vals, idx


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


__all__ = ["top_k", "cumsum"]
