"""Sampling API (mirror of tallax/_src/sampling.py and tallax/sampling.py).

`sample` is the vLLM-facing hook (sampling.py:331-343): one fused HIP kernel
does the per-row top-k (clamped to 128, as the reference's max_k=128), the
top-p filter, temperature and Gumbel-max draw.  `sample(..., max_k=K)`
with 128 < K <= 1024 opts into a wide-candidate kernel that honours per-row
top_k up to K instead of clamping it to 128.  `top_p_and_sample`
(sampling.py:210-269) runs the same tail on candidates the caller already
selected, and `top_p_mask` (sampling.py:25-62) only its top-p filter.

Operands are torch tensors on a ROCm device; the rng key is the two uint32
words of a threefry key (what `jax.random.key_data(key)` holds), as a device
tensor of dtype int32/uint32 or a host sequence of two ints.
"""
from __future__ import annotations

import numbers
from typing import Any, Sequence

import torch

from . import _lib

_SAMPLING_EPS = 1e-5  # sampling.py:22
NUM_CANDIDATES = 128  # the sampler's top-k width, max_k = NUM_LANES (sampling.py:283-290)
MAX_WIDE_CANDIDATES = 1024  # widest opt-in candidate list (tallax_sample_wide)


def _key_tensor(rng_key: Any, device: torch.device) -> torch.Tensor:
    if isinstance(rng_key, torch.Tensor):
        k = rng_key.reshape(-1)
        if k.numel() != 2:
            raise ValueError(f"rng_key must hold 2 uint32 words, got {k.numel()}")
        if k.dtype not in (torch.int32, torch.uint32):
            raise ValueError(f"rng_key dtype {k.dtype} must be int32 or uint32 key data")
        return k.to(device=device).view(torch.int32).contiguous()
    words = [int(w) & 0xFFFFFFFF for w in rng_key]
    if len(words) != 2:
        raise ValueError("rng_key must hold 2 uint32 words")
    words = [w - (1 << 32) if w >= (1 << 31) else w for w in words]
    return torch.tensor(words, dtype=torch.int32, device=device)


def _per_row(v: Any, rows: int, dtype: torch.dtype, device: torch.device) -> torch.Tensor:
    if isinstance(v, numbers.Number):
        # filled on the device: no host-to-device copy, so the call can be graph-captured
        return torch.full((rows,), v, dtype=dtype, device=device)
    t = v if isinstance(v, torch.Tensor) else torch.tensor(v, dtype=dtype)
    t = t.to(device=device, dtype=dtype)
    if t.ndim == 0:
        t = t.expand(rows)
    if t.shape != (rows,):
        raise ValueError(f"per-row parameter has shape {tuple(t.shape)}, expected ({rows},)")
    return t.contiguous()


def sample(rng_key: Any, logits: torch.Tensor, tpu_sampling_metadata: Any,
           *, replace_val: float = -1e12, dim0_offset: int = 0,
           workspace: torch.Tensor | None = None, max_k: int = NUM_CANDIDATES) -> torch.Tensor:
    """Fused top-k -> top-p -> temperature -> Gumbel-max sampler.

    Reference: sample(rng_key, logits, tpu_sampling_metadata) (sampling.py:331-343).
    `tpu_sampling_metadata` exposes `.top_k` (int, per row), `.top_p` and
    `.temperature` (float, per row).  The per-row k is clamped to 128 as in
    the reference (max_k=NUM_LANES, sampling.py:283-290).  Returns int32 [rows].

    max_k (opt-in, beyond the reference): the candidate width.  128 is the
    reference's; any value in [1, 1024] other than 128 runs the wide-candidate
    kernel, which is the same algorithm with the clamp at max_k (exact
    top-max_k, then top_p_and_sample over max_k candidates).
    """
    _lib.require_cuda(logits)
    if logits.ndim != 2:
        raise ValueError("Only 2D inputs supported")
    logits = logits.contiguous()
    rows, vocab = logits.shape
    dev = logits.device
    top_k = _per_row(tpu_sampling_metadata.top_k, rows, torch.int32, dev)
    top_p = _per_row(tpu_sampling_metadata.top_p, rows, torch.float32, dev)
    temp = _per_row(tpu_sampling_metadata.temperature, rows, torch.float32, dev)
    key = _key_tensor(rng_key, dev)
    dt = _lib.dtype_code(logits)
    if dt == _lib.I32:
        raise NotImplementedError("sample() needs float logits")
    out = torch.empty(rows, dtype=torch.int32, device=dev)
    if max_k != NUM_CANDIDATES:
        _wide_candidates(logits, dt, int(max_k), key, top_k, top_p, temp, dim0_offset, replace_val, out)
        return out
    need = _lib.LIB.tallax_sample_workspace_size(rows, vocab, dt)
    ws = _lib.workspace_arg(workspace, dev, need)
    _lib.check(_lib.LIB.tallax_fused_topk_topp_sample(
        logits.data_ptr(), dt, rows, vocab, top_k.data_ptr(), top_p.data_ptr(), temp.data_ptr(),
        key.data_ptr(), int(dim0_offset), float(replace_val), out.data_ptr(),
        ws.data_ptr() if need else None, ws.numel() if need else 0, _lib.stream_of(logits)),
        "sample")
    return out


def _wide_candidates(logits, dt, max_k, key, top_k, top_p, temp, dim0_offset, replace_val, out_tokens,
                     out_idx=None, out_vals=None):
    rows, vocab = logits.shape
    _lib.check(_lib.LIB.tallax_sample_wide(
        logits.data_ptr(), dt, rows, vocab, max_k,
        top_k.data_ptr() if top_k is not None else None, top_p.data_ptr() if top_p is not None else None,
        temp.data_ptr() if temp is not None else None, key.data_ptr() if key is not None else None,
        int(dim0_offset), float(replace_val),
        out_tokens.data_ptr() if out_tokens is not None else None,
        out_idx.data_ptr() if out_idx is not None else None,
        out_vals.data_ptr() if out_vals is not None else None, _lib.stream_of(logits)), "sample(max_k)")


def wide_top_k(logits: torch.Tensor, max_k: int) -> tuple[torch.Tensor, torch.Tensor]:
    """The candidates of sample(..., max_k): the max_k largest values of each
    row (value descending, ties to the lowest index; NaN, -inf and finfo.min
    reported as finfo(dtype).min), as float32 values and int32 columns
    [rows, max_k], before the per-row k mask.  max_k in [1, 1024]."""
    _lib.require_cuda(logits)
    if logits.ndim != 2:
        raise ValueError("Only 2D inputs supported")
    logits = logits.contiguous()
    dt = _lib.dtype_code(logits)
    if dt == _lib.I32:
        raise NotImplementedError("wide_top_k needs float logits")
    rows = logits.shape[0]
    vals = torch.empty((rows, max_k), dtype=torch.float32, device=logits.device)
    idx = torch.empty((rows, max_k), dtype=torch.int32, device=logits.device)
    _wide_candidates(logits, dt, int(max_k), None, None, None, None, 0, -1e12, None, idx, vals)
    return vals, idx


def top_p_mask(*, topk_logits: torch.Tensor, p: Any, replace_val: float, axis: int) -> torch.Tensor:
    """Top-p filter of descending candidates along axis 0.

    Reference: top_p_mask(*, topk_logits, p, replace_val, axis)
    (sampling.py:25-62).  topk_logits [k, B] float32, each column sorted
    descending, k <= 128 (the sampler's candidate count); p a scalar or [B].
    probs = softmax down each column, inclusive cumsum in the reference's tile
    order, t = #(cumsum < p); values >= the t-th (0.0 when t == k) are kept,
    ties included, the rest become replace_val.  Returns a new [k, B] tensor.
    Raises NotImplementedError for axis != 0, as the reference does.
    """
    if axis != 0:
        raise NotImplementedError("topp_mask only supports axis=0")
    _lib.require_cuda(topk_logits)
    if topk_logits.ndim != 2:
        raise ValueError("topk_logits must be 2D [k, batch]")
    if topk_logits.dtype != torch.float32:
        raise NotImplementedError("top_p_mask takes float32 candidates (the sampler casts to float32 first)")
    k, cols = topk_logits.shape
    dev = topk_logits.device
    logits = topk_logits.contiguous()
    tp = _per_row(p, cols, torch.float32, dev)
    out = torch.empty_like(logits)
    _lib.check(_lib.LIB.tallax_top_p_mask(logits.data_ptr(), k, cols, tp.data_ptr(), float(replace_val),
                                          out.data_ptr(), _lib.stream_of(logits)), "top_p_mask")
    return out


def top_p_and_sample(topk_logits: torch.Tensor, topk_idx: torch.Tensor, rng_key: Any,
                     top_p: Any, temperature: Any, *, vocab_size: int, replace_val: float,
                     interpret: bool = False, dim0_offset: int = 0) -> torch.Tensor:
    """Top-p filter, temperature and Gumbel-max draw over descending candidates.

    Reference: top_p_and_sample (sampling.py:210-269).  topk_logits [B, k]
    (k <= 128) sorted descending, topk_idx [B, k] int32 vocabulary ids.
    `interpret` is accepted for signature compatibility and ignored.
    """
    del interpret
    _lib.require_cuda(topk_logits, topk_idx)
    if topk_logits.ndim != 2 or topk_idx.shape != topk_logits.shape:
        raise ValueError("topk_logits and topk_idx must be 2D with the same shape")
    rows, k = topk_logits.shape
    dev = topk_logits.device
    logits = topk_logits.contiguous()
    idx = topk_idx.to(torch.int32).contiguous()
    tp = _per_row(top_p, rows, torch.float32, dev)
    tt = _per_row(temperature, rows, torch.float32, dev)
    key = _key_tensor(rng_key, dev)
    dt = _lib.dtype_code(logits)
    if dt == _lib.I32:
        raise NotImplementedError("top_p_and_sample needs float logits")
    out = torch.empty(rows, dtype=torch.int32, device=dev)
    _lib.check(_lib.LIB.tallax_top_p_and_sample(
        logits.data_ptr(), dt, idx.data_ptr(), rows, k, key.data_ptr(), tp.data_ptr(), tt.data_ptr(),
        int(vocab_size), float(replace_val), int(dim0_offset), out.data_ptr(), _lib.stream_of(logits)),
        "top_p_and_sample")
    return out


def sample_sharded(rng_key: Any, logit_shards: Sequence[torch.Tensor], tpu_sampling_metadata: Any,
                   *, replace_val: float = -1e12, dim0_offset: int = 0,
                   workspace: torch.Tensor | None = None) -> torch.Tensor:
    """`sample` over a vocabulary split into column shards, computed the way the
    reference's partitioned sampler does it, with every shard on this GPU.

    Reference: _top_k_with_sharding's partition (sampling.py:300-321) followed
    by top_p_and_sample (sampling.py:331-343).  Each shard [B, V_i] (V_i >= 128,
    consecutive column ranges in order) gives its sorted top-128 as composites
    in the global column frame (tallax_shard_candidates); the per-shard lists
    are stacked side by side (what the all-gather of a multi-GPU run
    delivers: [B, n, 128]); one kernel merges them into the global top-128
    (ties to the lowest global column, as in `sample`), writes replace_val
    (in the logits dtype) at positions >= top_k[row] and runs the sampler tail
    with vocab_size = sum(V_i) (tallax_sample_from_candidates).  The tokens
    equal `sample` on the concatenated logits.  Here every shard's step runs
    on this GPU at its real shape; in a multi-GPU run each GPU runs only its
    own, and the stacking is the collective.  At most 32 shards.  `workspace`:
    a uint8 device tensor large enough for the largest shard, used instead of
    the shared per-device buffer (the shard steps run in turn on one stream).
    """
    shards = list(logit_shards)
    if not shards:
        raise ValueError("sample_sharded needs at least one shard")
    if len(shards) > 32:
        raise NotImplementedError(f"{len(shards)} shards: at most 32 are supported")
    _lib.require_cuda(*shards)
    rows = shards[0].shape[0]
    for x in shards:
        if x.ndim != 2 or x.shape[0] != rows or x.dtype != shards[0].dtype or x.device != shards[0].device:
            raise ValueError("shards must be 2D [B, V_i] of one dtype and device with the same B")
    dev = shards[0].device
    dt = _lib.dtype_code(shards[0])
    if dt == _lib.I32:
        raise NotImplementedError("sample_sharded needs float logits")
    stream = _lib.stream_of(shards[0])
    lists, off = [], 0
    for x in shards:
        xc = x.contiguous()
        cols = xc.shape[1]
        need = _lib.LIB.tallax_shard_candidates_workspace_size(rows, cols, dt)
        ws = _lib.workspace_arg(workspace, dev, need)
        cand = torch.empty((rows, NUM_CANDIDATES), dtype=torch.int64, device=dev)
        _lib.check(_lib.LIB.tallax_shard_candidates(xc.data_ptr(), dt, rows, cols, off, cand.data_ptr(),
                                                    ws.data_ptr() if need else None, ws.numel() if need else 0,
                                                    stream), "sample_sharded (shard)")
        lists.append(cand)
        off += cols
    gathered = torch.stack(lists, 1)  # [B, n, 128]: the all-gather of a multi-GPU run
    top_k = _per_row(tpu_sampling_metadata.top_k, rows, torch.int32, dev)
    top_p = _per_row(tpu_sampling_metadata.top_p, rows, torch.float32, dev)
    temp = _per_row(tpu_sampling_metadata.temperature, rows, torch.float32, dev)
    key = _key_tensor(rng_key, dev)
    out = torch.empty(rows, dtype=torch.int32, device=dev)
    _lib.check(_lib.LIB.tallax_sample_from_candidates(
        gathered.data_ptr(), len(shards), dt, rows, off, top_k.data_ptr(), top_p.data_ptr(), temp.data_ptr(),
        key.data_ptr(), int(dim0_offset), float(replace_val), out.data_ptr(), stream), "sample_sharded (merge)")
    return out


class SamplingMetadata:
    """Minimal stand-in for vLLM's TPU sampling metadata (.top_k/.top_p/.temperature)."""

    def __init__(self, top_k: Any, top_p: Any, temperature: Any):
        self.top_k = top_k
        self.top_p = top_p
        self.temperature = temperature


__all__: Sequence[str] = ["sample", "wide_top_k", "sample_sharded", "top_p_mask", "top_p_and_sample", "SamplingMetadata"]
