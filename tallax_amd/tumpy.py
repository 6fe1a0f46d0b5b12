"""numpy-like API (mirror of tallax/tumpy.py: sort, argsort, take_along_axis).

Operands are torch tensors on a ROCm device; each op runs a gfx950 HIP
kernel through the C ABI in include/tallax_hip.h.
"""
from __future__ import annotations

import torch

from . import _lib


def take_along_axis(arr: torch.Tensor, indices: torch.Tensor, axis: int, interpret: bool = False) -> torch.Tensor:
    """out = arr[indices] along `axis` (0 or 1); 0 where an index is negative or
    out of range.

    Reference: tumpy.take_along_axis (tallax/tumpy.py:99-112) ->
    gather.take_along_axis (tallax/_src/gather.py:59-83).  2D operands; the
    batch extent (the other axis) must match.  Negative axes are normalised
    (the reference's `1 - axis` only works for 0 and 1).
    """
    del interpret
    _lib.require_cuda(arr, indices)
    if arr.ndim != 2 or indices.ndim != 2:
        raise ValueError("Only 2D inputs supported")
    axis = int(axis)
    if axis < 0:
        axis += 2
    if axis not in (0, 1):
        raise ValueError(f"axis {axis} out of range for a 2D operand")
    other = 1 - axis
    if arr.shape[other] != indices.shape[other]:
        raise ValueError(f"batch extents differ: {tuple(arr.shape)} vs {tuple(indices.shape)} along axis {other}")
    x = arr.contiguous()
    idx = indices.to(torch.int32).contiguous()
    dt = _lib.dtype_code(x)
    out = torch.empty(idx.shape, dtype=x.dtype, device=x.device)
    _lib.check(_lib.LIB.tallax_take_along_axis(x.data_ptr(), dt, x.shape[0], x.shape[1], idx.data_ptr(),
                                               idx.shape[0], idx.shape[1], axis, out.data_ptr(),
                                               _lib.stream_of(x)), "take_along_axis")
    return out


__all__ = ["take_along_axis"]
