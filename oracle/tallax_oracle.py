"""CPU oracle for the tallax sort / select / sample path -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import
this module, and only as the checker (or the timed CPU baseline).  The product
(`tallax_amd`) never imports it and has no CPU fallback.

Every function restates the reference (oliverdutton/tallax, read-only at
/root/reference) in numpy and cites the file:line it follows.  Float work is
done in numpy float32 with one IEEE operation per step, in the same order as
the HIP kernels, so GPU results are compared bit for bit.

Where the reference leaves a choice open (its tie order inside bitonic
networks, the summation order of XLA reductions, XLA's exp/log), the oracle
fixes the choice made by this build and says so; those parts are pinned by
closed forms and invariants in tests/, not by the reference:
  * top-k ties: lowest index first (the contract of BASELINE.json);
  * the softmax denominator in top_p_mask: a stride-halving tree over 128
    zero-padded slots; the per-tile sum inside cumsum: the pairwise tree
    that the tile's own Hillis-Steele scan produces;
  * exp/log: exp_f32/log_f32 below (<= 1 ulp, pinned against float64 numpy).
"""
from __future__ import annotations

import math

import numpy as np

F32 = np.float32
U32 = np.uint32
NUM_SUBLANES, NUM_LANES = 8, 128   # tallax/_src/utils.py:12-13

F32_MIN = F32(np.finfo(np.float32).min)
BF16_MIN = np.uint32(0xFF7F0000).view(np.float32)   # finfo(bfloat16).min widened to f32
TINY = np.finfo(np.float32).tiny


def _f(u: int) -> np.float32:
    return np.array(u, dtype=np.uint32).view(np.float32)[()]


# ---------------------------------------------------------------------------
# bf16 helpers (numpy has no bfloat16: bf16 arrays are carried as uint16 bits)
# ---------------------------------------------------------------------------
def bf16_bits_to_f32(bits: np.ndarray) -> np.ndarray:
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even float32 -> bfloat16 bits (NaN kept quiet)."""
    b = np.asarray(x, dtype=np.float32).view(np.uint32)
    nan = (b & 0x7FFFFFFF) > 0x7F800000
    r = (b + U32(0x7FFF) + ((b >> 16) & 1)) >> 16
    r = np.where(nan, (b | 0x00400000) >> 16, r)
    return r.astype(np.uint16)


def round_to_dtype(x, dtype: str) -> np.ndarray:
    x = np.asarray(x, dtype=np.float32)
    return bf16_bits_to_f32(f32_to_bf16_bits(x)) if dtype == "bf16" else x


I32_MIN = np.int32(np.iinfo(np.int32).min)


def dtype_min(dtype: str):
    """get_dtype_info(x).min (utils.py:48-56): finfo for floats, iinfo for int32."""
    if dtype == "i32":
        return I32_MIN
    return BF16_MIN if dtype == "bf16" else F32_MIN


def _as_values(x, dtype: str) -> np.ndarray:
    """Values as the oracle carries them: float32 (bf16 as its exact f32
    values) or int32."""
    return np.asarray(x, dtype=np.int32 if dtype == "i32" else np.float32)


def value_key(v: np.ndarray) -> np.ndarray:
    """Monotone int64 key of list values: select_key for floats (NaN lowest,
    -0 == +0), the value itself for int32."""
    v = np.asarray(v)
    if np.issubdtype(v.dtype, np.integer):
        return v.astype(np.int64)
    return select_key(v.astype(np.float32)).astype(np.int64)


# ---------------------------------------------------------------------------
# Keys (tallax/_src/utils.py:139-200) and the top-k composite order
# ---------------------------------------------------------------------------
def float_to_sortable_int(x: np.ndarray) -> np.ndarray:
    """standardize + float_to_sortable_int (utils.py:139-147,186-195):
    NaN -> bits 0x7FFFFFFE, -0 -> +0, negative floats -> i ^ 0x7FFFFFFF."""
    x = np.asarray(x, dtype=np.float32)
    i = x.view(np.int32).copy()
    i[np.isnan(x)] = 0x7FFFFFFE
    i[x == 0] = 0
    return np.where(i < 0, i ^ np.int32(0x7FFFFFFF), i).astype(np.int32)


def sortable_int_to_float(i: np.ndarray) -> np.ndarray:
    """utils.py:198-200."""
    i = np.asarray(i, dtype=np.int32)
    return np.where(i < 0, i ^ np.int32(0x7FFFFFFF), i).astype(np.int32).view(np.float32)


def select_key(x: np.ndarray) -> np.ndarray:
    """Unsigned key ordering values as the reference's strict-`>` top-k does
    (top_k.py:64): monotone in value, -0 == +0, NaN below -inf."""
    b = np.asarray(x, dtype=np.float32).view(np.uint32)
    a = b & U32(0x7FFFFFFF)
    k = np.where(b & U32(0x80000000), ~b, b | U32(0x80000000))
    k = np.where(a == 0, U32(0x80000000), k)
    k = np.where(a > U32(0x7F800000), U32(1), k)
    return k.astype(np.uint32)


def topk_composite(x: np.ndarray) -> np.ndarray:
    """u64 per element: select key << 32 | ~index; larger = earlier in the
    (value descending, index ascending) order."""
    k = select_key(x).astype(np.uint64)
    idx = np.arange(x.shape[-1], dtype=np.uint64)
    return (k << np.uint64(32)) | (np.uint64(0xFFFFFFFF) - idx)


def top_k(x: np.ndarray, k: int, dtype: str = "f32"):
    """Exact top-k along the last axis: the intended semantics of tax.top_k
    (top_k.py:516-567) under BASELINE's tie rule, i.e. the first k of
    xla_equivalent_sort(descending=True, is_stable=True) (sort.py:932-970).
    Elements the binned reference can never admit (<= finfo.min or NaN,
    top_k.py:64,241-243) are reported as finfo(dtype).min.
    x: float32 values (bf16 inputs as their exact f32 values), or int32 with
    dtype "i32": values descending, ties by lowest index, and iinfo.min (never
    admitted, the dtype's min) last in index order."""
    if dtype == "i32":
        xi = np.asarray(x, dtype=np.int32)
        key = (xi.astype(np.int64) + 2 ** 31).astype(np.uint64)
        comp = (key << np.uint64(32)) | (np.uint64(0xFFFFFFFF) - np.arange(xi.shape[-1], dtype=np.uint64))
        part = np.argpartition(comp, comp.shape[-1] - k, axis=-1)[..., -k:]
        order = np.argsort(np.take_along_axis(comp, part, -1), axis=-1)[..., ::-1]
        idx = np.take_along_axis(part, order, -1).astype(np.int32)
        return np.take_along_axis(xi, idx, -1).copy(), idx
    x = np.asarray(x, dtype=np.float32)
    comp = topk_composite(x)
    part = np.argpartition(comp, comp.shape[-1] - k, axis=-1)[..., -k:]
    order = np.argsort(np.take_along_axis(comp, part, -1), axis=-1)[..., ::-1]
    idx = np.take_along_axis(part, order, -1).astype(np.int32)
    vals = np.take_along_axis(x, idx, -1).copy()
    eligible = select_key(vals) > select_key(np.full((), dtype_min(dtype), np.float32))
    vals[~eligible] = dtype_min(dtype)
    return vals, idx


# ---------------------------------------------------------------------------
# approximate top-k: top_dynamic_k (tallax/_src/top_k.py:13-106, 203-514)
# and its schedule maths (tallax/top_k_convergence_theory.py:5-128)
# ---------------------------------------------------------------------------
def log2_ceil(x: int) -> int:
    """utils.log2 (utils.py:21-23): ceil(log2(x))."""
    return int(math.ceil(math.log2(x)))


def _log_convolve(log_a, log_b, trunc_len):
    ma, mb = np.max(log_a), np.max(log_b)
    if ma == -np.inf or mb == -np.inf:
        return np.full(min(len(log_a) + len(log_b) - 1, trunc_len), -np.inf)
    conv = np.convolve(np.exp(log_a - ma), np.exp(log_b - mb))[:trunc_len]
    with np.errstate(divide="ignore"):
        return np.log(conv) + ma + mb


def depth_probs(k: int, num_bins: int) -> np.ndarray:
    """compute_depth_probs (top_k_convergence_theory.py:45-103): P(max bin
    occupancy == m), m = 1..k, for k balls thrown uniformly into num_bins bins:
    P(max <= m) = k! / num_bins^k * [x^k] (sum_{i<=m} x^i / i!)^num_bins,
    the polynomial power taken by squaring in log space, truncated at x^k."""
    from scipy.special import gammaln
    log_fact_k = gammaln(k + 1)
    log_denom = k * np.log(num_bins)
    probs = np.zeros(k)
    prev = 0.0
    for m in range(1, k + 1):
        coeffs = -gammaln(np.arange(min(m + 1, k + 1)) + 1.0)
        cur, res, power = coeffs, np.array([0.0]), num_bins
        while power > 0:
            if power % 2 == 1:
                res = _log_convolve(res, cur, k + 1)
            if power > 1:
                cur = _log_convolve(cur, cur, k + 1)
            power //= 2
        log_cdf = (res[k] if len(res) > k else -np.inf) + log_fact_k - log_denom
        cdf = min(1.0, float(np.exp(log_cdf)) if log_cdf > -700 else 0.0)
        probs[m - 1] = max(0.0, cdf - prev)
        prev = cdf
        if cdf >= 1.0 - 1e-14:
            break
    return probs


def calculate_depth_thresholds(k, num_bins, block_size=8, target_yields=(0.66, 0.95, 0.9999)):
    """top_k_convergence_theory.py:106-128: the smallest depths d (1-based)
    with P(max occupancy <= d) ** block_size >= each target yield."""
    cdf = depth_probs(k, num_bins).cumsum()
    block = cdf ** block_size
    depths = set()
    for thr in target_yields:
        for i, val in enumerate(block):
            if val >= thr:
                depths.add(i + 1)
                break
    return tuple(sorted(depths))


def topm_schedule(max_k, num_bins, block_token, schedule=None):
    """top_dynamic_k's schedule (top_k.py:472-478): the auto schedule is the
    depth thresholds at yields (0.8, 0.98, 0.9999) plus one; deduplicated,
    sorted, with a leading 0."""
    if schedule is None:
        schedule = tuple(t + 1 for t in calculate_depth_thresholds(max_k, num_bins, block_token,
                                                                   target_yields=(0.8, 0.98, 0.9999)))
    return (0,) + tuple(sorted(set(int(m) for m in schedule)))


def binned_topm(x: np.ndarray, m: int, num_bins: int, dtype: str = "f32"):
    """binned_top_k (top_k.py:13-106) run to depth m: bin b holds columns
    j = b (mod num_bins); each bin keeps its m largest values; values <=
    finfo.min or NaN are never admitted.  The values at each rank are exactly
    those of the reference's strict-> sinking insert (pinned by a literal
    simulation in tests/test_oracle.py); among tied values the reference's
    kept indices depend on the insertion path, and this restatement keeps the
    lowest indices (the BASELINE tie contract).  Returns (vals [R, m, num_bins] f32, idxs
    [R, m, num_bins] int32), rank-major; unfilled slots hold (finfo.min, -1).
    int32 (dtype "i32"): bins start at iinfo.min, values and results int32."""
    x = _as_values(x, dtype)
    rows, cols = x.shape
    lo = dtype_min(dtype)
    nb = -(-cols // num_bins)
    pad = np.full((rows, nb * num_bins), lo if dtype == "i32" else np.nan, x.dtype)
    pad[:, :cols] = x
    vb = pad.reshape(rows, nb, num_bins)                        # [R, slice, bin]
    jb = (np.arange(nb)[:, None] * num_bins + np.arange(num_bins)[None, :]).astype(np.int64)
    admitted = vb > lo                                          # False for NaN, -inf, the dtype min, padding
    key = np.where(admitted, vb.astype(np.float64), -np.inf)    # exact for int32 too
    # order inside each bin: value descending, index ascending
    order = np.lexsort((np.broadcast_to(jb, vb.shape), -key), axis=1)[:, :m, :]
    vals = np.take_along_axis(key, order, axis=1)
    idxs = np.take_along_axis(np.broadcast_to(jb, vb.shape), order, axis=1)
    ok = vals > -np.inf
    out_v = np.full((rows, m, num_bins), lo, x.dtype)
    out_i = np.full((rows, m, num_bins), -1, np.int32)
    take = min(m, nb)
    out_v[:, :take][ok[:, :take]] = vals[:, :take][ok[:, :take]].astype(x.dtype)
    out_i[:, :take][ok[:, :take]] = idxs[:, :take][ok[:, :take]].astype(np.int32)
    return out_v, out_i


def list_order(v: np.ndarray, i: np.ndarray) -> np.ndarray:
    """Row-wise order of (value, index) list entries: select_key descending,
    then index ascending as an unsigned 32-bit number, so that the scratch
    fillers (finfo.min, index -1) follow every entry of a value >= finfo.min
    with a real index (the reference orders them by value; their indices are
    uninitialised there).  int32 values order by value."""
    key = value_key(v)
    iu = np.asarray(i).astype(np.int64) & 0xFFFFFFFF
    return np.lexsort((iu, -key), axis=-1)


def packed_bins(max_k: int, m: int) -> int:
    """num_packed_bins of _merge_unconverged_bins_top_k (top_k.py:122-124):
    the smallest power of two >= ceil(max_k / (m - 1))."""
    if m < 2:
        raise ValueError(f"the bin-packing merge needs a last schedule depth >= 2, got {m}")
    return 2 ** log2_ceil(-(-max_k // (m - 1)))


def merge_unconverged_bins(x, bv, bi, num_bins, m, max_k, dtype="f32"):
    """_merge_unconverged_bins_top_k (top_k.py:108-200) on the rows of one
    block, in place on their rank-major lists bv/bi [R, buf, num_bins]:
      * pivot = max over bins of rank m-1 (:126); per bin, the count of its
        ranks < m-1 that are >= pivot (:128-133);
      * the P = packed_bins(max_k, m) bins of the largest counts (:135-140;
        the reference's bitonic network leaves the order among equal counts
        open, and this restatement takes the lowest bin first);
      * every rank of a chosen bin becomes float32's finfo.min (:147-151,
        the scratch is 32-bit; iinfo(int32).min for int32) with its index kept;
      * packed position e of ceil(V / (128 num_bins / P)) * 128 holds column
        (e // P) * num_bins + chosen[e % P] (:153-183: lane L of packed tile
        j is slice j * 128 / P + L // P of bin chosen[L % P]); columns past
        the row hold (finfo(dtype).min, column), where the reference reads
        past the row's end;
      * rank 0 of bins 0..127 (the first 128 scratch columns) becomes the
        top-128 (list_order) of the packed entries and those 128 columns
        (:185-200).
    Needs num_bins % 128 == 0 (the first 128 columns are rank 0 of 128
    bins, and 128 bins are ranked at :139)."""
    if num_bins % NUM_LANES:
        raise NotImplementedError(f"the bin-packing merge needs num_bins % {NUM_LANES} == 0, got {num_bins}")
    x = _as_values(x, dtype)
    rows, V = x.shape
    P = packed_bins(max_k, m)
    lo = dtype_min(dtype)
    pivot = bv[:, m - 1, :].max(axis=1)
    cnt = (bv[:, :m - 1, :] >= pivot[:, None, None]).sum(axis=1)
    bins = np.broadcast_to(np.arange(num_bins), cnt.shape)
    chosen = np.lexsort((bins, -cnt), axis=1)[:, :P]
    for r in range(rows):
        bv[r][:, chosen[r]] = I32_MIN if dtype == "i32" else F32_MIN
    n = -(-V // (NUM_LANES * (num_bins // P))) * NUM_LANES
    e = np.arange(n)
    col = (e // P)[None, :] * num_bins + chosen[:, e % P]
    pv = np.where(col < V, np.take_along_axis(x, np.minimum(col, V - 1), 1), lo).astype(x.dtype)
    cv = np.concatenate([pv, bv[:, 0, :NUM_LANES]], axis=1)
    ci = np.concatenate([col.astype(np.int64), bi[:, 0, :NUM_LANES].astype(np.int64)], axis=1)
    top = list_order(cv, ci)[:, :NUM_LANES]
    bv[:, 0, :NUM_LANES] = np.take_along_axis(cv, top, 1)
    bi[:, 0, :NUM_LANES] = np.take_along_axis(ci, top, 1).astype(np.int32)


def top_dynamic_k(x, k, max_k, block_token=8, num_bins=128, schedule=None, replace_val=None,
                  dtype: str = "f32", guarantee_convergence: bool = False):
    """top_dynamic_k (top_k.py:203-514).  guarantee_convergence=False:
    (vals [R, max_k], idxs [R, max_k] int32, valid bool, depths [R] int32,
    cutoff_vals [R] f32); True: (vals, idxs).

    For each schedule step m (after the leading 0), evaluated while some row
    of the row's block of `block_token` rows has not converged:
      pivot = max over bins of the m-th largest, num_larger = #(ranks < m-1
      that are >= pivot); a row converges when num_larger >= k[row]; depth =
      m - 1 at the first convergence (max_k if never); cutoff = the pivot of
      the last step evaluated (top_k.py:283-320).
    With guarantee_convergence and a last depth other than max_k, a block
    that has not converged after its last step goes through
    merge_unconverged_bins (top_k.py:317-331).  The reference adds no max_k
    to the schedule, whatever its docstring says (top_k.py:444-450).
    valid = (max depth over all rows < schedule[-1]) or schedule[-1] == max_k.
    The output is the top-128 of the first depth_upper ranks of every bin,
    depth_upper the power-of-two bucket of the global max depth
    (top_k.py:333-364), in list_order (value, then lowest index: the
    reference's network order inside ties is not pinned), truncated to
    max_k and rounded to the dtype; positions >= k[row] get replace_val in
    the input dtype when given.
    Ranks at or past the m of a block's last evaluated step are never written
    for that block's rows: they keep the finfo.min the scratch starts with
    (top_k.py:241-243, 250-281), so they reach the output only as
    (finfo.min, -1) fillers (the reference leaves those indices
    uninitialised).
    int32 logits (dtype "i32"): int32 values and cutoff_vals (to_32bit_dtype,
    top_k.py:465); replace_val converted toward zero, saturated at the int32
    range."""
    x = _as_values(x, dtype)
    rows, cols = x.shape
    if rows % block_token:
        raise ValueError("num_tokens must be divisible by block_token")
    if max_k > NUM_LANES:
        raise NotImplementedError
    kk = np.broadcast_to(np.asarray(k, dtype=np.int64), (rows,))
    sched = topm_schedule(max_k, num_bins, block_token, schedule)
    max_m = sched[-1]
    merge = guarantee_convergence and max_m != max_k
    if merge:
        packed_bins(max_k, max_m)
        if num_bins % NUM_LANES:
            raise NotImplementedError(f"the bin-packing merge needs num_bins % {NUM_LANES} == 0")
    buf = max(max_m, 2 ** log2_ceil(max_m - 1)) if max_m > 1 else max_m
    bv, bi = binned_topm(x, buf, num_bins, dtype)
    lo = dtype_min(dtype)
    depths = np.full(rows, max_k, np.int32)
    cutoff = np.zeros(rows, np.int32 if dtype == "i32" else np.float32)
    for b0 in range(0, rows, block_token):
        blk = slice(b0, b0 + block_token)
        for m in sched[1:]:
            pivot = bv[blk, m - 1, :].max(axis=1)
            num_larger = (bv[blk, :m - 1, :] >= pivot[:, None, None]).sum(axis=(1, 2))
            conv = num_larger >= kk[blk]
            d = depths[blk]
            depths[blk] = np.where(conv & (d == max_k), m - 1, d)
            cutoff[blk] = pivot
            if conv.all():
                break
        # ranks >= m (the last step this block evaluated) were never written
        bv[blk, m:, :] = lo
        bi[blk, m:, :] = -1
        if merge and not conv.all():
            merge_unconverged_bins(x[blk], bv[blk], bi[blk], num_bins, max_m, max_k, dtype)
    gmax = int(depths.max())
    valid = bool(gmax < sched[-1] or sched[-1] == max_k)
    gsched = sorted(set(2 ** log2_ceil(s - 1) if s > 1 else s for s in sched))
    upper = gsched[-1]
    for lo_d, up_d in zip(gsched, gsched[1:]):
        if lo_d < gmax <= up_d:
            upper = up_d
            break
    sv = bv[:, :upper, :].reshape(rows, -1)
    si = bi[:, :upper, :].reshape(rows, -1)
    order = list_order(sv, si)[:, :NUM_LANES]
    vals = np.take_along_axis(sv, order, 1)[:, :max_k]
    vals = vals.copy() if dtype == "i32" else round_to_dtype(vals, dtype).astype(np.float32)
    idxs = np.take_along_axis(si, order, 1)[:, :max_k].copy()
    if replace_val is not None:
        pos = np.arange(vals.shape[1])[None, :]
        if dtype == "i32":
            r = 0.0 if math.isnan(replace_val) else min(max(float(replace_val), -2.0 ** 31), 2.0 ** 31 - 1)
            rv = np.int32(math.trunc(r))
        else:
            rv = round_to_dtype(np.float32(replace_val), dtype)
        vals = np.where(pos < kk[:, None], vals, rv).astype(vals.dtype)
    if guarantee_convergence:
        return vals, idxs
    return vals, idxs, valid, depths, cutoff


# ---------------------------------------------------------------------------
# exp / log (float32, one IEEE op per step; mirrors tallax_amd/csrc/tx_math.h)
# ---------------------------------------------------------------------------
_LOG2E, _LN2_HI, _LN2_LO = _f(0x3FB8AA3B), _f(0x3F317000), _f(0x3805FDF4)
_EXP_C = [_f(0x39500D01), _f(0x3AB60B61), _f(0x3C088889), _f(0x3D2AAAAB), _f(0x3E2AAAAB), F32(0.5)]
_LOG_C = [_f(0x3E1D89D9), _f(0x3E3A2E8C), _f(0x3E638E39), _f(0x3E924925), _f(0x3ECCCCCD), _f(0x3F2AAAAB)]
_SQRT2 = _f(0x3FB504F3)


def _pow2(n: np.ndarray) -> np.ndarray:
    return ((np.clip(n, -126, 127).astype(np.int32) + 127) << 23).astype(np.int32).view(np.float32)


def exp_f32(x) -> np.ndarray:
    """Cody-Waite reduction, exp(r) = 1 + (r + r^2 q(r)) (see tx_math.h)."""
    x = np.asarray(x, dtype=np.float32)
    with np.errstate(all="ignore"):
        xc = np.minimum(np.maximum(x, F32(-120.0)), F32(100.0))
        n = np.rint(xc * _LOG2E)
        r = (xc - n * _LN2_HI) - n * _LN2_LO
        q = np.full_like(r, _EXP_C[0])
        for c in _EXP_C[1:6]:
            q = q * r + c
        p = F32(1.0) + ((r * r) * q + r)
        ni = np.where(np.isnan(n), 0, n).astype(np.int32)
        normal = (ni >= -126) & (ni <= 127)
        n1 = np.where(ni < 0, -((-ni) // 2), ni // 2).astype(np.int32)
        n2 = ni - n1
        res = np.where(normal, p * _pow2(ni), (p * _pow2(n1)) * _pow2(n2))
        res = np.where(np.isnan(x), x, res)
    return res.astype(np.float32)


def log_f32(x) -> np.ndarray:
    """log via atanh series around 1 (see tx_math.h)."""
    x = np.asarray(x, dtype=np.float32)
    with np.errstate(all="ignore"):
        b = x.view(np.uint32)
        sub = b < U32(0x00800000)
        xs = np.where(sub, x * F32(8388608.0), x)
        bs = xs.view(np.uint32)
        e = np.where(sub, -23, 0).astype(np.int32) + (bs >> 23).astype(np.int32) - 127
        m = ((bs & U32(0x007FFFFF)) | U32(0x3F800000)).view(np.float32)
        big = m > _SQRT2
        m = np.where(big, m * F32(0.5), m)
        e = e + big.astype(np.int32)
        f = m - F32(1.0)
        s = f / (F32(2.0) + f)
        z = s * s
        R = np.full_like(z, _LOG_C[0])
        for c in _LOG_C[1:]:
            R = R * z + c
        R = R * z
        hfsq = (F32(0.5) * f) * f
        dk = e.astype(np.float32)
        res = dk * _LN2_HI - ((hfsq - (s * (hfsq + R) + dk * _LN2_LO)) - f)
        res = np.where(x == 0, F32(-np.inf), res)
        res = np.where(x == np.inf, F32(np.inf), res)
        res = np.where((x < 0) | np.isnan(x), F32(np.nan), res)
    return res.astype(np.float32)


# ---------------------------------------------------------------------------
# Threefry-2x32-20 and the sparse uniform (tallax/_src/sparse_random.py)
# ---------------------------------------------------------------------------
_ROT = (13, 15, 26, 6, 17, 29, 16, 24)


def threefry2x32(k0, k1, c0, c1):
    """Threefry-2x32, 20 rounds (Salmon et al., SC'11), elementwise over the
    counter arrays; JAX's threefry2x32_p (sparse_random.py:3,54)."""
    k0, k1 = U32(k0), U32(k1)
    c0 = np.asarray(c0, dtype=np.uint32)
    c1 = np.asarray(c1, dtype=np.uint32)
    ks = (k0, k1, U32(k0 ^ k1 ^ U32(0x1BD11BDA)))
    with np.errstate(over="ignore"):
        x0 = c0 + ks[0]
        x1 = c1 + ks[1]
        for blk in range(5):
            for i in range(4):
                r = _ROT[(blk & 1) * 4 + i]
                x0 = x0 + x1
                x1 = (x1 << U32(r)) | (x1 >> U32(32 - r))
                x1 = x1 ^ x0
            x0 = x0 + ks[(blk + 1) % 3]
            x1 = x1 + ks[(blk + 2) % 3] + U32(blk + 1)
    return x0.astype(np.uint32), x1.astype(np.uint32)


def bits_to_uniform(bits: np.ndarray) -> np.ndarray:
    """_bits_to_uniform (sparse_random.py:7-41) for float32."""
    bits = np.asarray(bits, dtype=np.uint32)
    return ((bits >> U32(9)) | U32(0x3F800000)).view(np.float32) - F32(1.0)


def sparse_random_uniform(key, indices, dim1_size, minval=0.0, maxval=1.0):
    """sparse_random_uniform (sparse_random.py:43-64): counter (hi=0,
    lo=row*dim1_size+col as uint32), bits = x0 ^ x1."""
    i0 = np.asarray(indices[0]).astype(np.int64)
    i1 = np.asarray(indices[1]).astype(np.int64)
    lo = ((i0 * int(dim1_size) + i1) & 0xFFFFFFFF).astype(np.uint32)
    o0, o1 = threefry2x32(key[0], key[1], np.zeros_like(lo), lo)
    f = bits_to_uniform(o0 ^ o1)
    mn, mx = F32(minval), F32(maxval)
    return np.maximum(mn, f * (mx - mn) + mn)


def gumbel(key, indices, dim1_size) -> np.ndarray:
    """-log(-log(u)), u from sparse_random_uniform(minval=tiny, maxval=1)
    (sparse_random.py:75-84)."""
    u = sparse_random_uniform(key, indices, dim1_size, minval=TINY, maxval=1.0)
    return -log_f32(-log_f32(u))


# ---------------------------------------------------------------------------
# max_arrays (bitonic_top_k.py:43-97): argmax tournament along axis 0
# ---------------------------------------------------------------------------
def max_arrays_axis0(operands):
    """Literal restatement of max_arrays(operands, num_keys=1, axis=0):
    pad dim0 to max(2^ceil(log2 n), 8) with dtype min, halve (left = first
    half, right = second half, keep left only if left > right), then the three
    in-tile xor stages (4, 2, 1).  Returns row 0 of every operand."""
    ops = [np.asarray(o) for o in operands]
    n = ops[0].shape[0]
    P = max(2 ** math.ceil(math.log2(n)), NUM_SUBLANES) if n > 1 else NUM_SUBLANES
    padded = []
    for o in ops:
        fill = np.finfo(o.dtype).min if np.issubdtype(o.dtype, np.floating) else np.iinfo(o.dtype).min
        pad = np.full((P - n,) + o.shape[1:], fill, dtype=o.dtype)
        padded.append(np.concatenate([o, pad], axis=0))
    ops = padded
    while ops[0].shape[0] > NUM_SUBLANES:
        h = ops[0].shape[0] // 2
        mask = ops[0][:h] > ops[0][h:]
        ops = [np.where(mask, o[:h], o[h:]) for o in ops]
    iota = np.arange(NUM_SUBLANES)
    for stage in (2, 1, 0):
        perm = iota ^ (1 << stage)
        mask = ops[0] > ops[0][perm]
        ops = [np.where(mask, o, o[perm]) for o in ops]
    return [o[0] for o in ops]


# ---------------------------------------------------------------------------
# cumsum (tallax/_src/cumsum.py:16-63)
# ---------------------------------------------------------------------------
def _hs_scan(t: np.ndarray, axis: int) -> np.ndarray:
    """Hillis-Steele inclusive scan inside one tile (cumsum.py:21-30)."""
    n = t.shape[axis]
    t = t.copy()
    s = 1
    while s < n:
        shifted = np.zeros_like(t)
        src = [slice(None)] * t.ndim
        dst = [slice(None)] * t.ndim
        src[axis] = slice(0, n - s)
        dst[axis] = slice(s, n)
        shifted[tuple(dst)] = t[tuple(src)]
        t = t + shifted
        s *= 2
    return t


def cumsum(arr: np.ndarray, axis: int, reverse: bool = False) -> np.ndarray:
    """cumsum_arrays (cumsum.py:32-63): pad to (8,128) tiles with 0, scan each
    tile (Hillis-Steele along `axis`), add the running total of earlier tiles
    (accumulated sequentially, tile sum = the tile's pairwise-tree sum), and
    for reverse flip tile order and in-tile order around the whole scan."""
    arr = np.asarray(arr)
    assert arr.ndim == 2 and axis in (0, 1)
    dt = arr.dtype
    rows, cols = arr.shape
    tr, tc = NUM_SUBLANES, NUM_LANES
    pr, pc = -(-rows // tr) * tr, -(-cols // tc) * tc
    a = np.zeros((pr, pc), dtype=dt)
    a[:rows, :cols] = arr
    tile = tr if axis == 0 else tc
    if reverse:
        a = np.flip(a, axis=axis)
    n = a.shape[axis] // tile
    with np.errstate(over="ignore"):
        tiles = np.split(a, n, axis=axis)
        outs = [_hs_scan(t, axis) for t in tiles]
        sums = [np.take(o, [tile - 1], axis=axis) for o in outs]   # pairwise-tree tile sums
        run = sums[0]
        for i in range(1, n):
            outs[i] = outs[i] + run
            run = run + sums[i]
        out = np.concatenate(outs, axis=axis)
    if reverse:
        out = np.flip(out, axis=axis)
    return np.ascontiguousarray(out[:rows, :cols]).astype(dt)


# ---------------------------------------------------------------------------
# sort (tallax/_src/sort.py:768-929, xla_equivalent_sort sort.py:932-970)
# ---------------------------------------------------------------------------
def sort(operands, num_keys: int, is_stable: bool = False, return_argsort: bool = False,
         descending: bool = False, dtypes=None):
    """tax.sort semantics on 2D numpy operands (float32 values, int32, or
    bfloat16 given as float32 values with dtypes[i] == "bf16").

    Order: lexicographic on the keys (floats standardised and compared as
    sortable ints, utils.py:139-195), then by original index: ascending in both
    directions when stable (sort.py:804-813,925-926; xla_equivalent_sort
    inserts -iota for descending), and for the packed bf16 + index path with a
    non-stable descending sort by descending index (the packed key is unique,
    utils.py:205-216).  Non-stable ties elsewhere follow the network and are
    not pinned by the reference; the ascending-index order is one valid
    outcome.  Returns (outputs tuple, path) with path "packed" or "unpacked";
    sorted float keys are decoded from the sortable ints (-0 -> +0, NaN ->
    0x7FFFFFFE, or bfloat16 0x7FFF on the packed path); bfloat16 keys come back
    as float32 on the unpacked path (utils.py:144-145 promotes them)."""
    ops = [np.asarray(o) for o in operands]
    dtypes = list(dtypes) if dtypes is not None else [("i32" if o.dtype == np.int32 else "f32") for o in ops]
    rows, cols = ops[0].shape
    if cols & (cols - 1) and any(d == "i32" for d in dtypes):
        is_stable = True                                        # sort.py:798-802
    use_indices = return_argsort or is_stable
    packed = dtypes[0] == "bf16" and len(ops) + int(use_indices) == 2 and use_indices and cols <= 65536
    ties_desc = packed and descending and not is_stable
    keys = []
    for i in range(num_keys):
        k = ops[i].astype(np.int32) if dtypes[i] == "i32" else float_to_sortable_int(ops[i].astype(np.float32))
        k = k.astype(np.int64)
        keys.append(-k if descending else k)
    idx = np.broadcast_to(np.arange(cols, dtype=np.int64), (rows, cols))
    tie = -idx if ties_desc else idx
    perm = np.empty((rows, cols), dtype=np.int64)
    for r in range(rows):
        perm[r] = np.lexsort([tie[r]] + [k[r] for k in reversed(keys)])
    outs = []
    for i, o in enumerate(ops):
        g = np.take_along_axis(o, perm, axis=1)
        if i < num_keys and dtypes[i] != "i32":
            g = sortable_int_to_float(float_to_sortable_int(g.astype(np.float32)))
            if packed:
                g = (g.view(np.uint32) & U32(0xFFFF0000)).view(np.float32)   # bf16 result, NaN 0x7FFF
        outs.append(g)
    if return_argsort:
        outs.append(perm.astype(np.int32))
    return tuple(outs), ("packed" if packed else "unpacked")


# ---------------------------------------------------------------------------
# config 5: softmax -> top-k -> cumsum -> top-p cutoff
# ---------------------------------------------------------------------------
def softmax_topk_cumsum_f64(x: np.ndarray, k: int, p: float):
    """The float64 truth for the composition jax.nn.softmax, tax.sort(probs,
    descending=True, return_argsort=True)[:, :k], tax.cumsum(axis=1) and
    #(cumsum < p): (idx [R, k] int32, probs64, cum64, cutoff64).  Positions are
    the k largest logits, ties to the lowest index (probability is monotone in
    the logit, so this is the descending probability order with equal
    probabilities in a valid order)."""
    x = np.asarray(x, dtype=np.float32)
    comp = topk_composite(x)
    part = np.argpartition(comp, comp.shape[-1] - k, axis=-1)[..., -k:]
    order = np.argsort(np.take_along_axis(comp, part, -1), axis=-1)[..., ::-1]
    idx = np.take_along_axis(part, order, -1).astype(np.int32)
    x64 = x.astype(np.float64)
    m = x64.max(axis=1, keepdims=True)
    with np.errstate(invalid="ignore"):
        e = np.exp(x64 - m)
    probs = np.take_along_axis(e, idx, 1) / e.sum(axis=1, keepdims=True)
    cum = np.cumsum(probs, axis=1)
    return idx, probs, cum, (cum < p).sum(axis=1).astype(np.int32)


# ---------------------------------------------------------------------------
# take_along_axis (tallax/_src/gather.py:11-83)
# ---------------------------------------------------------------------------
def take_along_axis(values: np.ndarray, indices: np.ndarray, axis: int) -> np.ndarray:
    """take_along_axis_arrays (gather.py:11-45): out = values[idx] along
    `axis` where 0 <= idx < extent, else 0 (the accumulators start at zero
    and only in-range tiles overwrite them; no negative wrap)."""
    values = np.asarray(values)
    idx = np.asarray(indices).astype(np.int64)
    assert values.ndim == 2 and idx.ndim == 2 and axis in (0, 1)
    ext = values.shape[axis]
    ok = (idx >= 0) & (idx < ext)
    safe = np.where(ok, idx, 0)
    if ext == 0:
        return np.zeros(idx.shape, dtype=values.dtype)
    got = np.take_along_axis(values, safe, axis=axis)
    return np.where(ok, got, np.zeros((), dtype=values.dtype)).astype(values.dtype)


# ---------------------------------------------------------------------------
# top_p_mask / top_p_and_sample / sample (tallax/_src/sampling.py)
# ---------------------------------------------------------------------------
def _tree_width(k: int) -> int:
    """Slots of the top-p sum tree: 128 for the reference's k <= 128; the
    next power of two for the wide-candidate sampler's k <= 1024 (beyond the
    reference, whose sampler never has more than 128 candidates)."""
    w = 128
    while w < k:
        w *= 2
    return w


def _tree_sum_axis0(e: np.ndarray) -> np.ndarray:
    """Sum over axis 0 as a stride-halving tree over _tree_width(k) (128 for
    k <= 128) zero-padded slots: x[:64] + x[64:], then x[:32] + x[32:], ..."""
    k = e.shape[0]
    x = np.zeros((_tree_width(k),) + e.shape[1:], dtype=np.float32)
    x[:k] = e
    while x.shape[0] > 1:
        h = x.shape[0] // 2
        x = x[:h] + x[h:]
    return x


def top_p_mask(topk_logits: np.ndarray, p: np.ndarray, replace_val: float) -> np.ndarray:
    """top_p_mask(axis=0) (sampling.py:25-62) on [k, B] descending candidates."""
    L = np.asarray(topk_logits, dtype=np.float32)
    k = L.shape[0]
    with np.errstate(all="ignore"):
        e = exp_f32(L - L[:1])
        s = _tree_sum_axis0(e)
        probs = e / s
    c = cumsum(probs, axis=0)
    t = (c < np.asarray(p, dtype=np.float32)[None, :]).sum(0)
    # take_along_axis_arrays: out-of-range index (t == k) gathers 0 (gather.py:11-45)
    thr = np.where(t < k, L[np.minimum(t, k - 1), np.arange(L.shape[1])], F32(0.0))
    return np.where(L >= thr[None, :], L, F32(replace_val)).astype(np.float32)


def top_p_and_sample(topk_logits, topk_idx, key, top_p, temperature, vocab_size,
                     replace_val, dim0_offset: int = 0) -> np.ndarray:
    """top_p_and_sample_arrays (sampling.py:65-115): [B, k] -> [B] tokens."""
    L = np.asarray(topk_logits, dtype=np.float32).T
    I = np.asarray(topk_idx, dtype=np.int32).T
    B = L.shape[1]
    top_p = np.broadcast_to(np.asarray(top_p, dtype=np.float32), (B,))
    temperature = np.broadcast_to(np.asarray(temperature, dtype=np.float32), (B,))
    masked = top_p_mask(L, top_p, replace_val)
    with np.errstate(all="ignore"):
        scaled = masked / temperature[None, :]
        batch = np.broadcast_to(np.arange(B, dtype=np.int64)[None, :] + dim0_offset, L.shape)
        g = gumbel(key, (batch, I), vocab_size)
        score = scaled + g
    _, tok = max_arrays_axis0([score, I])
    greedy = I[0]
    return np.where(temperature < F32(1e-5), greedy, tok).astype(np.int32)


def sample(key, logits, top_k_per_row, top_p, temperature, dtype: str = "f32",
           replace_val: float = -1e12, dim0_offset: int = 0, max_k: int = NUM_LANES) -> np.ndarray:
    """sample() (sampling.py:331-343) on one device: exact top-128 (per-row k
    mask with replace_val in the logits dtype, top_k.py:365-369), then
    top_p_and_sample with replace_val.  max_k != 128 is the wide-candidate
    sampler (beyond the reference): the same steps with max_k candidates."""
    x = np.asarray(logits, dtype=np.float32)
    vals, idx = top_k(x, max_k, dtype)
    kr = np.asarray(top_k_per_row, dtype=np.int64)
    rv = round_to_dtype(F32(replace_val), dtype)
    vals = np.where(np.arange(max_k)[None, :] < kr[:, None], vals, rv)
    return top_p_and_sample(vals, idx, key, top_p, temperature, x.shape[1], replace_val, dim0_offset)
