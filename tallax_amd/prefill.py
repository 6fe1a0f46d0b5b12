"""Prefill-scale softmax -> top-k -> cumsum -> top-p cutoff.

The reference runs this as a composition: jax.nn.softmax over the vocabulary,
tax.sort(probs, num_keys=1, descending=True, return_argsort=True) cut to the
first k columns (tallax/_src/sort.py:768-929), tax.cumsum(axis=1)
(tallax/_src/cumsum.py:75-101) and the count of cumsum < p.  Here it is one
gfx950 kernel reading the logits from HBM once (include/tallax_hip.h:
tallax_softmax_topk_cumsum).
"""
from __future__ import annotations

import torch

from . import _lib


def softmax_topk_cumsum(logits: torch.Tensor, k: int = 2048, p: float = 0.9):
    """Returns (probs [R, k] f32 descending, idx [R, k] int32, cumsum [R, k]
    f32, cutoff [R] int32 = #(cumsum < p)).

    The positions are the k largest logits with ties to the lowest index (the
    descending probability order, equal probabilities in a valid order);
    probabilities are float32 softmax values (sum order of the kernel, within
    1e-5 relative of float64); the cumsum follows tax.cumsum's tile order.
    """
    _lib.require_cuda(logits)
    if logits.ndim != 2:
        raise ValueError("Only 2D inputs supported")
    if logits.dtype != torch.float32:
        raise NotImplementedError("softmax_topk_cumsum takes float32 logits")
    x = logits.contiguous()
    rows, cols = x.shape
    k = int(k)
    dev = x.device
    probs = torch.empty((rows, k), dtype=torch.float32, device=dev)
    idx = torch.empty((rows, k), dtype=torch.int32, device=dev)
    cum = torch.empty((rows, k), dtype=torch.float32, device=dev)
    cutoff = torch.empty(rows, dtype=torch.int32, device=dev)
    _lib.check(_lib.LIB.tallax_softmax_topk_cumsum(x.data_ptr(), rows, cols, k, float(p), probs.data_ptr(),
                                                   idx.data_ptr(), cum.data_ptr(), cutoff.data_ptr(),
                                                   _lib.stream_of(x)), "softmax_topk_cumsum")
    return probs, idx, cum, cutoff


__all__ = ["softmax_topk_cumsum"]
