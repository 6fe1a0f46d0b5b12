"""numpy-like API (mirror of tallax/tumpy.py: sort, argsort, take_along_axis).

Operands are torch tensors on a ROCm device; each op runs a gfx950 HIP
kernel through the C ABI in include/tallax_hip.h.
"""
from __future__ import annotations

import torch

from . import _lib


def _rows_view(a: torch.Tensor, axis):
    if axis is None:
        work = a.reshape(-1)
        return work.reshape(1, -1), tuple(work.shape)
    ndim = a.ndim
    canonical = axis if axis >= 0 else axis + ndim
    if canonical != ndim - 1:
        raise ValueError("tumpy only supports sorting along the last axis.")
    return a.reshape(-1, a.shape[-1]), tuple(a.shape)


def sort(a: torch.Tensor, axis=-1, kind=None, order=None, stable: bool = True, descending: bool = False,
         interpret: bool = False) -> torch.Tensor:
    """Sorted copy along the last axis (or of the flattened array, axis=None).

    Reference: tumpy.sort (tallax/tumpy.py:6-52) -> tax.sort(num_keys=1,
    is_stable=stable, return_argsort=False).  `kind` and `order` are ignored.
    """
    del kind, order, interpret
    from . import tax
    a2, shape = _rows_view(a, axis)
    (out,) = tax.sort(a2, num_keys=1, is_stable=stable, descending=descending, return_argsort=False)
    return out.reshape(shape)


def argsort(a: torch.Tensor, axis=-1, kind=None, order=None, stable: bool = True, descending: bool = False,
            interpret: bool = False) -> torch.Tensor:
    """int32 indices that sort `a` along the last axis (or flattened).

    Reference: tumpy.argsort (tallax/tumpy.py:54-97) -> tax.sort(num_keys=1,
    is_stable=stable, return_argsort=True).
    """
    del kind, order, interpret
    from . import tax
    a2, shape = _rows_view(a, axis)
    _, idx = tax.sort(a2, num_keys=1, is_stable=stable, descending=descending, return_argsort=True)
    return idx.reshape(shape)


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


__all__ = ["sort", "argsort", "take_along_axis"]
