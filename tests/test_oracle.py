"""Pins the CPU oracle (oracle/tallax_oracle.py) before it is trusted as the
GPU checker: known-answer vectors, an independent implementation (rocRAND),
float64 numpy, closed forms, brute force and statistics."""
import json
import math
import os
import shutil
import subprocess

import numpy as np
import pytest

from oracle import tallax_oracle as O

HERE = os.path.dirname(os.path.abspath(__file__))


# --------------------------------------------------------------------------- threefry
def test_threefry_known_answers():
    with open(os.path.join(HERE, "golden", "threefry_kat.json")) as f:
        kat = json.load(f)["vectors"]
    for v in kat:
        k0, k1 = (int(x, 16) for x in v["key"])
        c0, c1 = (int(x, 16) for x in v["counter"])
        o0, o1 = O.threefry2x32(k0, k1, c0, c1)
        assert (int(o0), int(o1)) == tuple(int(x, 16) for x in v["out"])


@pytest.mark.skipif(shutil.which("/opt/rocm/bin/hipcc") is None, reason="hipcc absent")
def test_threefry_matches_rocrand(tmp_path):
    exe = tmp_path / "tf"
    subprocess.run(["/opt/rocm/bin/hipcc", "-O1", os.path.join(HERE, "golden", "rocrand_threefry_check.cpp"),
                    "-o", str(exe)], check=True, capture_output=True)
    rng = np.random.default_rng(7)
    q = rng.integers(0, 2**32, size=(2000, 4), dtype=np.uint64).astype(np.uint32)
    inp = "\n".join(" ".join(f"{int(v):08x}" for v in row) for row in q) + "\n"
    out = subprocess.run([str(exe)], input=inp, capture_output=True, text=True, check=True).stdout.split()
    ref = np.array([int(x, 16) for x in out], dtype=np.uint64).reshape(-1, 2).astype(np.uint32)
    mine = np.stack([np.array([int(a) for a in O.threefry2x32(r[0], r[1], r[2], r[3])]) for r in q[:200]])
    assert np.array_equal(mine, ref[:200])
    # vectorised path over the remaining rows (one key per call)
    for r, exp in zip(q[200:400], ref[200:400]):
        o0, o1 = O.threefry2x32(r[0], r[1], np.array([r[2]]), np.array([r[3]]))
        assert (int(o0[0]), int(o1[0])) == (int(exp[0]), int(exp[1]))


def test_bits_to_uniform_closed_form():
    b = np.array([0, 0x1FF, 0x200, 0xFFFFFFFF, 0x80000000], dtype=np.uint32)
    u = O.bits_to_uniform(b)
    assert u[0] == 0.0 and u[1] == 0.0
    assert u[2] == np.float32(2.0**-23)
    assert u[3] == np.float32(1 - 2.0**-23)
    assert u[4] == np.float32(0.5)
    # u = max(tiny, f + tiny): f == 0 -> tiny, otherwise f itself (tiny is far below f's ulp)
    g = O.sparse_random_uniform((0, 1), (np.zeros(1000, np.int64), np.arange(1000)), 1000,
                                minval=O.TINY, maxval=1.0)
    f = O.bits_to_uniform(np.bitwise_xor(*O.threefry2x32(0, 1, np.zeros(1000, np.uint32),
                                                        np.arange(1000, dtype=np.uint32))))
    assert np.array_equal(g, np.where(f == 0, np.float32(O.TINY), f))


def test_sparse_counter_layout():
    # counter = row * dim1_size + col (sparse_random.py:49-50), hi word 0
    key = (0, 42)
    rows = np.array([0, 3, 7]); cols = np.array([5, 0, 255])
    u = O.sparse_random_uniform(key, (rows, cols), 256)
    o0, o1 = O.threefry2x32(0, 42, np.zeros(3, np.uint32), (rows * 256 + cols).astype(np.uint32))
    assert np.array_equal(u, O.bits_to_uniform(o0 ^ o1))


# --------------------------------------------------------------------------- exp / log
def _ulp_err(got, want64):
    want = want64.astype(np.float32)
    ok = np.isfinite(want) & (want != 0)
    sp = np.spacing(np.abs(want[ok])).astype(np.float64)
    return np.abs(got[ok].astype(np.float64) - want64[ok]) / sp


def test_exp_accuracy_and_specials():
    rng = np.random.default_rng(1)
    x = np.concatenate([rng.uniform(-103.9, 88.7, 400000), rng.uniform(-1, 1, 100000),
                        rng.uniform(-30, 0, 100000)]).astype(np.float32)
    e = O.exp_f32(x)
    err = _ulp_err(e, np.exp(x.astype(np.float64)))
    assert err.max() <= 1.0, err.max()
    assert O.exp_f32(np.float32(0)) == 1.0
    assert O.exp_f32(np.float32(-np.inf)) == 0.0
    assert O.exp_f32(np.float32(np.inf)) == np.inf
    assert O.exp_f32(np.float32(89.0)) == np.inf
    assert O.exp_f32(np.float32(-104.0)) == 0.0
    assert np.isnan(O.exp_f32(np.float32(np.nan)))
    # subnormal results: within one subnormal step of the float64 value
    xs = np.linspace(-103.0, -87.5, 5000).astype(np.float32)
    es = O.exp_f32(xs).astype(np.float64)
    assert np.max(np.abs(es - np.exp(xs.astype(np.float64)))) <= 2.0**-149


def test_log_accuracy_and_specials():
    rng = np.random.default_rng(2)
    bits = rng.integers(1, 0x7F800000, 500000, dtype=np.uint64).astype(np.uint32)  # all positive finite
    x = np.concatenate([bits.view(np.float32), rng.uniform(0.5, 2.0, 200000).astype(np.float32),
                        rng.uniform(0, 1, 200000).astype(np.float32)])
    x = x[x > 0]
    l = O.log_f32(x)
    err = _ulp_err(l, np.log(x.astype(np.float64)))
    assert err.max() <= 1.0, err.max()
    assert O.log_f32(np.float32(1.0)) == 0.0
    assert O.log_f32(np.float32(0.0)) == -np.inf
    assert O.log_f32(np.float32(np.inf)) == np.inf
    assert np.isnan(O.log_f32(np.float32(-1.0)))
    for k in range(-149, 128, 7):
        v = np.float32(2.0**k)
        assert O.log_f32(v) == np.float32(k * np.log(2.0))


# --------------------------------------------------------------------------- max_arrays tie rule
def _bitrev(p, bits):
    return int(format(p, f"0{bits}b")[::-1], 2)


@pytest.mark.parametrize("n", [8, 16, 50, 64, 128])
def test_max_arrays_tie_rule_is_bit_reversed_position(n):
    """The literal tournament of max_arrays (bitonic_top_k.py:43-97) keeps, among
    tied maxima, the position with the largest bit-reversed index over
    log2(padded n) bits; without ties it is the plain argmax.  The HIP sampler
    implements the bit-reversal rule directly."""
    rng = np.random.default_rng(n)
    P = max(2 ** int(np.ceil(np.log2(n))), 8)
    bits = int(np.log2(P))
    scores = rng.integers(0, 4, size=(n, 3000)).astype(np.float32)
    pos = np.broadcast_to(np.arange(n, dtype=np.int32)[:, None], scores.shape)
    _, win = O.max_arrays_axis0([scores, pos])
    for b in range(scores.shape[1]):
        m = scores[:, b].max()
        cands = [p for p in range(n) if scores[p, b] == m]
        assert win[b] == max(cands, key=lambda p: _bitrev(p, bits))
    uniq = rng.standard_normal((n, 500)).astype(np.float32)
    _, win = O.max_arrays_axis0([uniq, np.broadcast_to(np.arange(n, dtype=np.int32)[:, None], uniq.shape)])
    assert np.array_equal(win, uniq.argmax(0))


# --------------------------------------------------------------------------- top-k
def _brute_topk(row, k, dmin):
    keyed = []
    for i, v in enumerate(row):
        if np.isnan(v):
            rank_v = -np.inf; nan = True
        else:
            rank_v = float(v); nan = False
        keyed.append((0 if nan else 1, 0.0 if v == 0 else rank_v, -i))
    order = sorted(range(len(row)), key=lambda i: keyed[i], reverse=True)[:k]
    vals = np.array([row[i] for i in order], dtype=np.float32)
    elig = np.array([(not np.isnan(v)) and v > dmin for v in vals])
    vals[~elig] = dmin
    return vals, np.array(order, dtype=np.int32)


def test_topk_oracle_brute_force_with_ties_nan_inf():
    rng = np.random.default_rng(3)
    for trial in range(60):
        n = int(rng.integers(1, 40)); k = int(rng.integers(1, n + 1))
        row = rng.integers(-3, 4, n).astype(np.float32)
        special = rng.random(n)
        row[special < 0.1] = np.nan
        row[(special >= 0.1) & (special < 0.2)] = -np.inf
        row[(special >= 0.2) & (special < 0.3)] = -0.0
        row[(special >= 0.3) & (special < 0.35)] = np.float32(np.finfo(np.float32).min)
        v, i = O.top_k(row[None], k)
        bv, bi = _brute_topk(row, k, O.F32_MIN)
        assert np.array_equal(i[0], bi), (row, k)
        assert np.array_equal(v[0].view(np.uint32), bv.view(np.uint32))


def test_topk_oracle_matches_stable_sort_closed_form():
    rng = np.random.default_rng(4)
    x = (rng.standard_normal((16, 3000)) * 4).round().astype(np.float32)  # heavy ties
    v, i = O.top_k(x, 100)
    ref_i = np.argsort(-x, axis=1, kind="stable")[:, :100]
    assert np.array_equal(i, ref_i)
    assert np.array_equal(v, np.take_along_axis(x, ref_i, 1))


# --------------------------------------------------------------------------- cumsum
@pytest.mark.parametrize("shape", [(8, 128), (16, 256), (128, 8), (256, 16), (13, 167)])
@pytest.mark.parametrize("axis", [0, 1])
@pytest.mark.parametrize("reverse", [False, True])
def test_cumsum_oracle(shape, axis, reverse):
    """tests/cumsum_test.py of the reference: float within rtol 1e-3/atol 1e-6
    of lax.cumsum, int exact.  Here against float64/int64 numpy."""
    rng = np.random.default_rng(42)
    xf = rng.standard_normal(shape).astype(np.float32)
    xi = rng.integers(0, 100, shape).astype(np.int32)
    def ref(a):
        a = np.flip(a, axis) if reverse else a
        r = np.cumsum(a.astype(np.float64 if a.dtype.kind == "f" else np.int64), axis=axis)
        return np.flip(r, axis) if reverse else r
    got = O.cumsum(xf, axis, reverse)
    assert got.dtype == np.float32
    np.testing.assert_allclose(got, ref(xf), rtol=1e-5, atol=1e-5)
    assert np.array_equal(O.cumsum(xi, axis, reverse), ref(xi).astype(np.int32))


def test_cumsum_tile_sum_is_pairwise_tree():
    rng = np.random.default_rng(5)
    t = rng.standard_normal((8, 128)).astype(np.float32)
    hs = O._hs_scan(t, 1)
    x = t.copy()
    while x.shape[1] > 1:  # adjacent pairs, then pairs of pairs
        x = x[:, 0::2] + x[:, 1::2]
    assert np.array_equal(hs[:, -1], x[:, 0])


# --------------------------------------------------------------------------- top-p and sampling
def test_top_p_mask_invariants():
    rng = np.random.default_rng(6)
    L = -np.sort(-rng.standard_normal((64, 300)).astype(np.float32) * 2, axis=0)
    p = rng.uniform(0.05, 0.99, 300).astype(np.float32)
    m = O.top_p_mask(L, p, -1e12)
    kept = m > -1e11
    assert kept[0].all()                                   # the top candidate always survives
    assert np.all(np.diff(kept.astype(int), axis=0) <= 0)  # kept set is a prefix
    # float64 restatement: kept count = (#cumsum < p) + 1 (+ ties), away from rounding edges
    pr = np.exp(L.astype(np.float64) - L[0]); pr /= pr.sum(0)
    cum = np.cumsum(pr, 0)
    t = (cum < p).sum(0)
    thr = L[np.minimum(t, 63), np.arange(300)]
    want = (L >= thr).sum(0)
    close = np.abs(cum - p).min(0) < 1e-5
    assert np.array_equal(kept.sum(0)[~close], want[~close])
    # p tiny keeps exactly the ties of the maximum
    m0 = O.top_p_mask(L, np.full(300, 1e-9, np.float32), -1e12)
    assert np.array_equal((m0 > -1e11).sum(0), (L == L[0]).sum(0))


def test_sampler_greedy_and_k1():
    rng = np.random.default_rng(7)
    x = rng.standard_normal((32, 4096)).astype(np.float32) * 3
    argmax = np.argsort(-x, axis=1, kind="stable")[:, 0]
    t = O.sample((0, 1), x, np.full(32, 50), np.full(32, 0.9, np.float32), np.full(32, 1e-6, np.float32))
    assert np.array_equal(t, argmax)
    t = O.sample((0, 1), x, np.full(32, 1), np.full(32, 0.9, np.float32), np.full(32, 1.0, np.float32))
    assert np.array_equal(t, argmax)


def test_sampler_distribution_is_softmax_of_filtered_logits():
    """Gumbel-max over the kept candidates draws token j with probability
    softmax(logits/T)[j] (chi-square, 20000 independent rows)."""
    B = 20000
    logits = np.array([2.0, 1.5, 1.0, 0.5, 0.0, -0.5, -1.0, -3.0], dtype=np.float32)
    L = np.broadcast_to(logits, (B, 8))
    I = np.broadcast_to(np.arange(8, dtype=np.int32) * 3, (B, 8))
    T = np.full(B, 0.7, np.float32)
    p = np.full(B, 0.95, np.float32)
    tok = O.top_p_and_sample(L, I, (0, 99), p, T, vocab_size=24, replace_val=-1e12)
    pr = np.exp(logits.astype(np.float64) - 2); pr /= pr.sum()
    cut = int((np.cumsum(pr) < 0.95).sum())
    kept = logits >= logits[cut]
    q = np.exp(np.where(kept, logits / 0.7, -np.inf) - 2 / 0.7); q /= q.sum()
    counts = np.bincount(tok // 3, minlength=8)
    assert counts[~kept].sum() == 0
    exp_c = q[kept] * B
    chi2 = ((counts[kept] - exp_c) ** 2 / exp_c).sum()
    assert chi2 < 30.0, (counts, exp_c)  # dof <= 7, p ~ 1e-4


def test_sampler_replace_and_quirk_threshold_zero():
    # k-mask replaces positions >= k with replace_val in the logits dtype
    assert O.round_to_dtype(np.float32(-1e12), "bf16").view(np.uint32) == 0xD3690000
    # top-p with cumsum never reaching p: threshold gathers 0 (out-of-range take)
    L = np.array([[3.0], [2.0], [1.0], [-1.0]], dtype=np.float32)
    m = O.top_p_mask(L, np.array([1.5], np.float32), -1e12)
    assert np.array_equal(m[:, 0], np.array([3.0, 2.0, 1.0, -1e12], np.float32))


def test_wide_sampler_oracle_dense_brute_force():
    """sample(max_k=K) (beyond the reference's 128) against a dense
    restatement: the top-K set by a stable sort, the k mask, a float64 top-p
    cut (rows whose cumsum lies within 1e-4 of p are skipped), then
    argmax(masked / T + gumbel(row, token)) over the whole vocabulary."""
    rng = np.random.default_rng(21)
    B, V, K = 12, 3000, 700
    x = (rng.standard_normal((B, V)) * 2).astype(np.float32)
    x[:, ::7] = np.round(x[:, ::7])  # ties
    kr = rng.integers(150, K + 1, B)
    p = rng.uniform(0.3, 0.95, B).astype(np.float32)
    T = rng.uniform(0.5, 1.5, B).astype(np.float32)
    tok = O.sample((3, 4), x, kr, p, T, max_k=K)
    checked = 0
    for b in range(B):
        order = np.argsort(-x[b].astype(np.float64), kind="stable")[:K]
        v = x[b, order].astype(np.float64)
        v[kr[b]:] = -1e12
        pr = np.exp(v - v[0]); pr /= pr.sum()
        c = np.cumsum(pr)
        if np.min(np.abs(c - p[b])) < 1e-4:
            continue
        t = int((c < p[b]).sum())
        keep = v >= v[t]
        g = O.gumbel((3, 4), (np.full(K, b), order.astype(np.int32)), V).astype(np.float64)
        score = np.where(keep, v, -1e12) / T[b] + g
        assert tok[b] == order[np.argmax(score)], b
        checked += 1
    assert checked >= 8


def test_wide_sampler_oracle_reduces_to_the_reference_width():
    """With every per-row k <= 128, widening the candidate list only adds
    masked candidates: sample(max_k=K) == sample() for any K >= 128."""
    rng = np.random.default_rng(22)
    B, V = 16, 5000
    x = (rng.standard_normal((B, V)) * 3).astype(np.float32)
    kr = rng.integers(1, 129, B)
    p = rng.uniform(0.5, 1.0, B).astype(np.float32)
    p[::5] = 1.0
    T = rng.uniform(0.5, 1.5, B).astype(np.float32)
    want = O.sample((9, 1), x, kr, p, T)
    for K in (200, 512, 1024):
        assert np.array_equal(O.sample((9, 1), x, kr, p, T, max_k=K), want), K


# --------------------------------------------------------------------------- take_along_axis
def test_take_along_axis_oracle_closed_form():
    """gather.py:11-45: in-range indices gather exactly as numpy does; negative
    and out-of-range ones give 0 (no wrap), on both axes."""
    rng = np.random.default_rng(3)
    v = rng.standard_normal((6, 50)).astype(np.float32)
    idx = rng.integers(0, 50, (6, 70)).astype(np.int32)
    assert np.array_equal(O.take_along_axis(v, idx, 1), np.take_along_axis(v, idx, 1))
    idx2 = idx.copy()
    idx2[:, ::3] = -1
    idx2[:, 1::5] = 50
    got = O.take_along_axis(v, idx2, 1)
    bad = (idx2 < 0) | (idx2 >= 50)
    assert np.all(got[bad] == 0) and np.array_equal(got[~bad], np.take_along_axis(v, idx2 % 50, 1)[~bad])
    vt = v.T.copy()
    assert np.array_equal(O.take_along_axis(vt, idx.T.copy(), 0), np.take_along_axis(vt, idx.T, 0))
    iv = rng.integers(-100, 100, (4, 9)).astype(np.int32)
    assert O.take_along_axis(iv, np.full((4, 2), 9, np.int32), 1).dtype == np.int32


# --------------------------------------------------------------------------- sort
def test_sort_oracle_matches_stable_argsort_and_torch():
    """Stable ascending / descending orders equal np.argsort(kind="stable") on
    the sortable keys and torch.sort(stable=True) on NaN-free data; descending
    stable equals xla_equivalent_sort's (-iota key, then reverse) construction
    (sort.py:955-969)."""
    import torch
    rng = np.random.default_rng(21)
    x = np.round(rng.standard_normal((6, 300)) * 4).astype(np.float32) / 4     # many ties
    (v, i), path = O.sort([x], 1, is_stable=True, return_argsort=True)
    assert path == "unpacked"
    assert np.array_equal(i, np.argsort(x, axis=1, kind="stable"))
    tv, ti = torch.sort(torch.from_numpy(x), dim=1, stable=True)
    assert np.array_equal(i, ti.numpy()) and np.array_equal(v, tv.numpy())
    (vd, idd), _ = O.sort([x], 1, is_stable=True, return_argsort=True, descending=True)
    # xla_equivalent_sort: lexsort ascending on (x, -iota), then reverse
    cols = x.shape[1]
    for r in range(x.shape[0]):
        o = np.lexsort([-np.arange(cols), x[r]])[::-1]
        assert np.array_equal(idd[r], o)
    td, tdi = torch.sort(torch.from_numpy(x), dim=1, descending=True, stable=True)
    assert np.array_equal(idd, tdi.numpy())


def test_sort_oracle_key_decode_and_paths():
    """S1: NaN sorts above +inf and decodes to 0x7FFFFFFE, -0 decodes to +0;
    bf16 keys come back as float32 unpacked, bf16 (NaN 0x7FFF) packed."""
    x = np.array([[1.0, np.nan, -0.0, np.inf, -np.inf, 0.0, -2.5, np.nan]], np.float32)
    (v,), _ = O.sort([x], 1)
    b = v.view(np.uint32)[0]
    assert list(b[:3]) == [0xFF800000, 0xC0200000, 0]          # -inf, -2.5, +0 (was -0 or +0)
    assert b[3] == 0 and b[5] == 0x7F800000 and b[6] == b[7] == 0x7FFFFFFE
    xb = O.round_to_dtype(x, "bf16")
    (vb, ib), path = O.sort([xb], 1, is_stable=True, return_argsort=True, dtypes=["bf16"])
    assert path == "packed"
    assert vb.view(np.uint32)[0, -1] == 0x7FFF0000 and vb.view(np.uint32)[0, 2] == 0
    (vu,), path = O.sort([xb], 1, is_stable=False, dtypes=["bf16"])
    assert path == "unpacked" and vu.view(np.uint32)[0, -1] == 0x7FFFFFFE


def test_sort_oracle_packed_descending_nonstable_ties():
    """The packed bf16+index key is unique, so a non-stable descending argsort
    has ties in descending index order (utils.py:205-216); stable keeps them
    ascending (sort.py:807-809)."""
    x = np.array([[1.0, 2.0, 1.0, 2.0, 1.0]], np.float32)
    (_, i_ns), _ = O.sort([x], 1, is_stable=False, return_argsort=True, descending=True, dtypes=["bf16"])
    (_, i_st), _ = O.sort([x], 1, is_stable=True, return_argsort=True, descending=True, dtypes=["bf16"])
    assert list(i_ns[0]) == [3, 1, 4, 2, 0]
    assert list(i_st[0]) == [1, 3, 0, 2, 4]


def test_sort_oracle_two_keys_and_forced_stable():
    rng = np.random.default_rng(4)
    k0 = rng.integers(0, 3, (3, 50)).astype(np.int32)       # non-power-of-two int keys: forced stable
    k1 = rng.integers(0, 4, (3, 50)).astype(np.float32)
    pay = rng.standard_normal((3, 50)).astype(np.float32)
    (a, b, c), _ = O.sort([k0, k1, pay], 2)
    for r in range(3):
        o = np.lexsort([np.arange(50), k1[r], k0[r]])
        assert np.array_equal(c[r], pay[r, o]) and np.array_equal(a[r], k0[r, o])


@pytest.mark.parametrize("descending", [False, True])
def test_sort_oracle_many_keys_brute_force(descending):
    """Three keys, lexicographic (sort.py:768-929, S1-S2), against Python's
    sorted() on tuples: float keys standardised (NaN above +inf, -0 == +0),
    ties by ascending index in both directions; key outputs decoded."""
    rng = np.random.default_rng(40 + descending)
    n = 60
    k0 = rng.integers(-2, 2, (2, n)).astype(np.int32)
    k1 = rng.integers(-2, 2, (2, n)).astype(np.float32)
    k1[0, ::9] = np.nan
    k1[1, ::4] = -0.0
    k2 = np.round(rng.standard_normal((2, n))).astype(np.float32)
    pay = rng.standard_normal((2, n)).astype(np.float32)
    (a, b, c, d, perm), _ = O.sort([k0, k1, k2, pay], 3, is_stable=True, return_argsort=True,
                                   descending=descending)

    def std(x):  # standardised order of a float key
        x = float(x)
        return math.inf * 2 if x != x else (0.0 if x == 0.0 else x)

    sign = -1 if descending else 1
    for r in range(2):
        o = sorted(range(n), key=lambda j: (sign * int(k0[r, j]), sign * std(k1[r, j]), sign * std(k2[r, j]), j))
        assert np.array_equal(perm[r], np.array(o, dtype=np.int32))
        assert np.array_equal(d[r], pay[r, o]) and np.array_equal(a[r], k0[r, o])
        got_k1 = b[r]
        assert np.all(np.isnan(got_k1) == np.isnan(k1[r, o]))
        assert np.array_equal(got_k1.view(np.uint32) == 0x80000000, np.zeros(n, bool))  # no -0 left


# --------------------------------------------------------------------------- approximate top-k
def test_depth_probs_closed_forms_and_monte_carlo():
    """compute_depth_probs (top_k_convergence_theory.py:45-103): P(max bin
    occupancy == m) for k balls in n bins.  Closed forms for tiny cases and a
    Monte Carlo estimate for a realistic one; the product's restatement
    (tallax_amd/schedule.py) agrees with the oracle's."""
    from tallax_amd import schedule as S
    assert np.allclose(O.depth_probs(1, 128), [1.0])
    assert np.allclose(O.depth_probs(2, 2), [0.5, 0.5])
    assert np.allclose(O.depth_probs(3, 3), [6 / 27, 18 / 27, 3 / 27])
    rng = np.random.default_rng(0)
    k, n, trials = 50, 128, 20000
    occ = np.zeros((trials, n), np.int32)
    balls = rng.integers(0, n, (trials, k))
    np.add.at(occ, (np.repeat(np.arange(trials), k), balls.ravel()), 1)
    mc = np.bincount(occ.max(1), minlength=k + 1)[1:] / trials
    p = O.depth_probs(k, n)
    assert np.abs(np.cumsum(mc) - np.cumsum(p)).max() < 0.015
    for kk, nn in [(50, 128), (128, 256), (8, 16), (1, 128)]:
        assert np.allclose(S.max_occupancy_pdf(kk, nn), O.depth_probs(kk, nn), rtol=1e-9, atol=1e-12)
        assert S.topm_schedule(kk, nn, 8) == O.topm_schedule(kk, nn, 8)[1:]


def _exact_max_occupancy_cdf(k: int, n: int, m_max: int | None = None) -> list:
    """P(max bin occupancy <= m) for m = 1..k, k labelled balls thrown into n
    bins, as exact fractions: N_m / n^k, where N_m counts the maps
    [k] -> [n] with every bin holding <= m balls.  N_m = k! [x^k]
    (sum_{i<=m} x^i / i!)^n; with integer coefficients c_j = j! [x^j] the
    product of two such series is the binomial convolution
    c_j = sum_i C(j, i) a_i b_{j-i}, so the power is taken by repeated
    squaring over Python integers, truncated at degree k.  Independent of
    the log-space float routine it checks."""
    from fractions import Fraction

    def bconv(a, b):
        return [sum(math.comb(j, i) * a[i] * b[j - i] for i in range(j + 1)) for j in range(k + 1)]

    out = []
    for m in range(1, (m_max or k) + 1):
        base = [1 if j <= m else 0 for j in range(k + 1)]
        acc = [1] + [0] * k
        p = n
        while p:
            if p & 1:
                acc = bconv(acc, base)
            base = bconv(base, base)
            p >>= 1
        out.append(Fraction(acc[k], n ** k))
    return out


def _exact_schedule(k: int, n: int, block: int, yields=(0.8, 0.98, 0.9999)) -> tuple:
    """top_dynamic_k's automatic schedule (top_k.py:444-450) from the exact
    cdf: for each yield, the first depth m with cdf(m)^block >= yield
    (top_k_convergence_theory.py:115-125, 1-based), then + 1, deduplicated
    and sorted.  The yields are compared as the float64 values the reference
    passes, converted exactly."""
    from fractions import Fraction
    cdf = _exact_max_occupancy_cdf(k, n, min(k, 12))   # every yield here is met by depth 12
    depths = set()
    for y in yields:
        for m, c in enumerate(cdf, start=1):
            if c ** block >= Fraction(y):
                depths.add(m)
                break
        else:
            raise AssertionError(f"yield {y} not met by depth {len(cdf)}")
    return tuple(sorted(d + 1 for d in depths))


def test_depth_schedule_exact_rational():
    """calculate_depth_thresholds + the +1 of top_dynamic_k
    (top_k_convergence_theory.py:103-128, top_k.py:444-450), pinned by exact
    rational arithmetic rather than a second log-space restatement.

    Hand-checkable cases first, each exercising one step:
      * k = 1: one ball, max occupancy is always 1, so every yield is met at
        depth 1 and the schedule is (2,) -- the "+1";
      * k = 3, n = 3: 27 maps; max <= 1 for the 3! = 6 permutations (2/9),
        max <= 2 for all but the 3 maps into one bin (8/9), max <= 3 always.
        block 1: yield 0.8 first met at depth 2, 0.98 and 0.9999 at depth 3
        -> thresholds (2, 3), schedule (3, 4) -- the "first index" and the
        deduplication; block 8: (8/9)^8 = 0.39 < 0.8, so only depth 3 ->
        schedule (4,) -- the "cdf ** block" power;
      * k = 2, n = 2: max <= 1 with probability 1/2, so a yield of 0.4 is met
        at depth 1 with block 1 but at depth 2 with block 2 (1/4 < 0.4).
    Then realistic cases against the exact counts, both restatements (the
    oracle's and the product's tallax_amd/schedule.py) checked against them.
    """
    from fractions import Fraction
    from tallax_amd import schedule as S
    assert _exact_max_occupancy_cdf(3, 3) == [Fraction(2, 9), Fraction(8, 9), Fraction(1)]
    assert _exact_max_occupancy_cdf(2, 2) == [Fraction(1, 2), Fraction(1)]
    assert _exact_max_occupancy_cdf(1, 128) == [Fraction(1)]
    hand = {(1, 128, 8): (2,), (3, 3, 1): (3, 4), (3, 3, 8): (4,)}
    for (k, n, b), want in hand.items():
        assert _exact_schedule(k, n, b) == want
        assert O.topm_schedule(k, n, b)[1:] == want, (k, n, b)
        assert S.topm_schedule(k, n, b) == want, (k, n, b)
    assert _exact_schedule(2, 2, 1, yields=(0.4,)) == (2,)
    assert _exact_schedule(2, 2, 2, yields=(0.4,)) == (3,)
    assert O.calculate_depth_thresholds(2, 2, 1, (0.4,)) == (1,)
    assert O.calculate_depth_thresholds(2, 2, 2, (0.4,)) == (2,)
    assert S.calculate_depth_thresholds(2, 2, 1, (0.4,)) == (1,)
    assert S.calculate_depth_thresholds(2, 2, 2, (0.4,)) == (2,)
    realistic = {(50, 128, 8): (5, 6, 8), (128, 256, 8): (6, 7, 9), (64, 128, 8): (5, 6, 8),
                 (8, 16, 8): (4, 5, 7), (16, 32, 8): (5, 6, 7), (32, 64, 8): (5, 6, 8)}
    for (k, n, b), want in realistic.items():
        assert _exact_schedule(k, n, b) == want, (k, n, b)
        assert O.topm_schedule(k, n, b)[1:] == want, (k, n, b)
        assert S.topm_schedule(k, n, b) == want, (k, n, b)
    # the cdf itself: float restatements within 1e-9 of the exact fractions
    for k, n in [(50, 128), (16, 32)]:
        exact = np.array([float(c) for c in _exact_max_occupancy_cdf(k, n, 12)])
        for pdf in (O.depth_probs(k, n), S.max_occupancy_pdf(k, n)):
            got = np.cumsum(pdf)
            m = min(len(got), len(exact))
            assert np.abs(got[:m] - exact[:m]).max() < 1e-9


def test_binned_topm_brute_force():
    """binned_top_k (top_k.py:13-106) simulated literally (strict-> sinking
    insert in index order; NaN / -inf / finfo.min never admitted): the values at
    every rank equal the oracle's per-bin top-m exactly.  The indices agree
    wherever the value is untied; among tied values the reference's kept
    indices depend on the insertion path (a displaced element cannot pass an
    equal one), so the oracle's lowest-index choice is the documented
    contract there."""
    rng = np.random.default_rng(8)
    x = np.round(rng.standard_normal((3, 70)) * 2).astype(np.float32) / 2
    x[0, ::7] = np.nan
    x[1, ::5] = -np.inf
    x[2, ::3] = O.F32_MIN
    x[:, 60:] = rng.standard_normal((3, 10)).astype(np.float32) * 7    # some untied values
    v, i = O.binned_topm(x, 4, 8)
    for r in range(3):
        for b in range(8):
            lv, li = [O.F32_MIN] * 4, [-1] * 4
            for j in range(b, 70, 8):
                bv, bi = x[r, j], j
                for q in range(4):
                    if bv > lv[q]:
                        lv[q], bv = bv, lv[q]
                        li[q], bi = bi, li[q]
            assert np.array_equal(v[r, :, b], np.array(lv, np.float32))
            col = x[r, b::8]
            for q in range(4):
                if li[q] >= 0 and np.sum(col == lv[q]) == 1:
                    assert i[r, q, b] == li[q]


def test_int32_topk_brute_force():
    """int32 top-k (dtype-generic reference: iinfo bins, utils.py:48-56): the
    oracle equals a brute-force sort by (value descending, index ascending),
    with iinfo.min -- never admitted, the dtype's min -- last in index order;
    also on heavy ties (randint(0, 1000), bitonic_topk_test.py:20-23)."""
    rng = np.random.default_rng(21)
    imin, imax = np.iinfo(np.int32).min, np.iinfo(np.int32).max
    for trial in range(60):
        n = int(rng.integers(1, 60)); k = int(rng.integers(1, n + 1))
        row = rng.integers(-4, 5, n).astype(np.int32)
        sp = rng.random(n)
        row[sp < 0.15] = imin
        row[(sp >= 0.15) & (sp < 0.25)] = imax
        order = sorted(range(n), key=lambda j: (-int(row[j]), j))[:k]
        v, i = O.top_k(row[None], k, "i32")
        assert v.dtype == np.int32 and np.array_equal(i[0], np.array(order, np.int32))
        assert np.array_equal(v[0], row[order])
    x = rng.integers(0, 1000, (13, 167)).astype(np.int32)
    v, i = O.top_k(x, 128, "i32")
    for r in range(13):
        order = sorted(range(167), key=lambda j: (-int(x[r, j]), j))[:128]
        assert np.array_equal(i[r], order) and np.array_equal(v[r], x[r, order])


def test_int32_binned_topm_literal():
    """binned_top_k on int32 simulated literally (strict-> sinking insert from
    iinfo.min): values at every rank equal the oracle's, and indices where the
    value is untied in its bin."""
    rng = np.random.default_rng(22)
    imin = np.iinfo(np.int32).min
    x = rng.integers(-6, 7, (3, 90)).astype(np.int32)
    x[0, ::7] = imin
    x[1, 60:] = rng.integers(-2 ** 31 + 1, 2 ** 31 - 1, 30).astype(np.int32)   # untied values
    v, i = O.binned_topm(x, 5, 8, "i32")
    assert v.dtype == np.int32
    for r in range(3):
        for b in range(8):
            lv, li = [imin] * 5, [-1] * 5
            for j in range(b, 90, 8):
                bv, bi = int(x[r, j]), j
                for q in range(5):
                    if bv > lv[q]:
                        lv[q], bv = bv, lv[q]
                        li[q], bi = bi, li[q]
            assert np.array_equal(v[r, :, b], np.array(lv, np.int32))
            col = x[r, b::8]
            for q in range(5):
                if li[q] >= 0 and np.sum(col == lv[q]) == 1:
                    assert i[r, q, b] == li[q]


def _int32_dyn_cases():
    rng = np.random.default_rng(78)
    imin = np.iinfo(np.int32).min
    x = rng.integers(-2 ** 31 + 1, 2 ** 31 - 1, (16, 3000), dtype=np.int64).astype(np.int32)  # untied
    for r in (5, 6):                       # block 0 cannot converge: 40 spikes in bin 0
        x[r, rng.choice(3000 // 64, 40, replace=False) * 64] = 2 ** 31 - 1 - rng.permutation(40)
    x[9, ::3] = imin
    yield "int32 unconverged block", x, rng.integers(1, 33, 16).astype(np.int32), 32, 8, 64, (3, 6, 12), False
    yield "int32 merge, P = 8", x, rng.integers(1, 33, 16).astype(np.int32), 32, 8, 128, (3, 6), True
    y = np.full((8, 700), imin, np.int32)
    for r in range(8):                     # a few admissible values per row
        y[r, rng.choice(700, 6 + r, replace=False)] = rng.integers(-1000, 1000, 6 + r)
    yield "int32 mostly iinfo.min rows", y, rng.integers(1, 17, 8).astype(np.int32), 16, 4, 32, (2, 5), False


@pytest.mark.parametrize("replace", [None, -1e12, 7.9])
@pytest.mark.parametrize("case", list(_int32_dyn_cases()), ids=lambda c: c[0] if isinstance(c, tuple) else str(c))
def test_int32_top_dynamic_k_matches_literal_restatement(case, replace):
    """int32 logits: every output of O.top_dynamic_k(dtype="i32") equals the
    literal block restatement run on the int32 scratch (iinfo.min bins and
    merge fill, int32 cutoff_vals, replace_val stored into int32)."""
    _, x, k, max_k, bt, nb, sched, gc = case
    (lv, li), lvalid, ld, lc = _literal_dynamic_top_k(x, k, max_k, bt, nb, sched, replace, "i32",
                                                      guarantee_convergence=gc)
    out = O.top_dynamic_k(x, k, max_k, block_token=bt, num_bins=nb, schedule=sched, replace_val=replace,
                          dtype="i32", guarantee_convergence=gc)
    ov, oi = out[:2]
    assert ov.dtype == np.int32
    assert np.array_equal(oi, li) and np.array_equal(ov, lv)
    if not gc:
        _, _, ovalid, od, oc = out
        assert oc.dtype == np.int32
        assert ovalid == lvalid and np.array_equal(od, ld) and np.array_equal(oc, lc)


def test_top_dynamic_k_converged_rows_are_exact():
    rng = np.random.default_rng(2)
    x = rng.standard_normal((16, 20000)).astype(np.float32)
    x[3, rng.choice(20000, 40, replace=False)] = 8.0        # ties inside the top-k
    vals, idx, valid, depths, cutoff = O.top_dynamic_k(x, 50, 50)
    ev, ei = O.top_k(x, 50)
    assert valid and (depths < 50).all()
    assert np.array_equal(vals, ev) and np.array_equal(idx, ei)
    # cutoff is a pivot: a value present in the row, below every kept value
    assert all(cutoff[r] in x[r] and cutoff[r] <= vals[r, -1] for r in range(16))
    # an unconvergeable schedule: depth stays max_k, valid is False, result approximate
    v2, i2, valid2, d2, _ = O.top_dynamic_k(x, 50, 50, schedule=(2,))
    assert not valid2 and (d2 == 50).all()
    assert np.all(np.diff(v2, axis=1) <= 0)


# A literal restatement of dynamic_top_k_refs (top_k.py:203-370) and its
# wrapper (top_k.py:433-514), block by block, used only to pin the oracle:
# scratch values start at finfo.min for each block (:241-243) and indices are
# uninitialised (here the sentinel _GARBAGE); each schedule step runs
# binned_top_k (:13-106) with the completed ranks invalidated by index
# (:53-60) and a strict-> sinking insert (:61-72), only while the block's
# termination flag is 0 (:250-315); the final top-128 reads the first
# depth_upper * num_bins scratch columns (:333-364); replace_val at positions
# >= k (:365-369).  The final order among equal values is the lowest index
# (BASELINE's tie contract; the reference's network order is unpinned).
_GARBAGE = 2 ** 31 - 1


def _literal_dynamic_top_k(x, k, max_k, block_token, num_bins, schedule, replace_val=None, dtype="f32",
                           guarantee_convergence=False):
    rows, vocab = x.shape
    lo = O.dtype_min(dtype)
    vt = np.int32 if dtype == "i32" else np.float32              # to_32bit_dtype of the scratch (:476-478)
    kk = np.broadcast_to(np.asarray(k, np.int64), (rows,))
    sched = (0,) + tuple(sorted(set(schedule)))
    max_m = sched[-1]
    buf = max(max_m, 2 ** O.log2_ceil(max_m - 1)) * num_bins
    sv = np.full((rows, buf), 0 if dtype == "i32" else np.nan, vt)
    si = np.full((rows, buf), _GARBAGE, np.int64)
    depths = np.zeros(rows, np.int32)
    cutoff = np.zeros(rows, vt)
    nslices = -(-vocab // num_bins)
    xp = np.full((rows, nslices * num_bins), lo, vt)            # pad(val='min'), :96-105
    xp[:, :vocab] = x
    for pid in range(rows // block_token):
        ts = slice(pid * block_token, (pid + 1) * block_token)
        sv[ts] = lo
        depths[ts] = max_k
        flag = 0
        for completed, m in zip(sched, sched[1:]):
            if flag != 0:
                continue
            vals = [sv[ts, i * num_bins:(i + 1) * num_bins].copy() for i in range(m)]
            idxs = [si[ts, i * num_bins:(i + 1) * num_bins].copy() for i in range(m)]
            for s in range(nslices):
                bv = xp[ts, s * num_bins:(s + 1) * num_bins].copy()
                bi = np.broadcast_to(s * num_bins + np.arange(num_bins), bv.shape).astype(np.int64).copy()
                for i in range(completed):
                    bv = np.where(bi == idxs[i], lo, bv)
                for i in range(completed, m):
                    mask = bv > vals[i]
                    vals[i], bv = np.where(mask, bv, vals[i]), np.where(mask, vals[i], bv)
                    idxs[i], bi = np.where(mask, bi, idxs[i]), np.where(mask, idxs[i], bi)
            for i in range(completed, m):
                sv[ts, i * num_bins:(i + 1) * num_bins] = vals[i]
                si[ts, i * num_bins:(i + 1) * num_bins] = idxs[i]
            pivot = vals[m - 1].max(-1)
            num_larger = sum((v >= pivot[:, None]) for v in vals[:m - 1]).sum(-1) if m > 1 else np.zeros(block_token)
            flag = 0
            for i in range(block_token):
                r = pid * block_token + i
                contains = num_larger[i] >= kk[r]
                flag += int(contains)
                if contains and depths[r] == max_k:
                    depths[r] = m - 1
                cutoff[r] = pivot[i]
            if flag != block_token:
                flag = 0
        if guarantee_convergence and max_m != max_k and flag == 0:    # :317-331
            _literal_merge(x[ts], sv, si, ts, num_bins, max_m, max_k, dtype)
    gts = sorted(set(2 ** O.log2_ceil(s - 1) if s > 1 else s for s in sched))
    gmax = int(depths.max())
    valid = bool(gmax < sched[-1] or sched[-1] == max_k)
    out = None
    for d_lo, d_up in zip(gts, gts[1:]):
        if (d_lo < gmax <= d_up) or (d_up == gts[-1] and gmax > d_up):
            v = sv[:, :d_up * num_bins].astype(np.float64)
            i = si[:, :d_up * num_bins]
            order = np.lexsort((i, -v), axis=1)[:, :128]
            ov = np.take_along_axis(sv[:, :d_up * num_bins], order, 1)
            if dtype != "i32":
                ov = O.round_to_dtype(ov, dtype)
            oi = np.take_along_axis(i, order, 1)
            if replace_val is not None:
                if dtype == "i32":     # stored into int32: toward zero, saturated
                    rv = np.int32(math.trunc(min(max(float(replace_val), -2.0 ** 31), 2.0 ** 31 - 1)))
                else:
                    rv = O.round_to_dtype(np.float32(replace_val), dtype)
                ov = np.where(np.arange(ov.shape[1])[None, :] < kk[:, None], ov, rv).astype(vt)
            oi = np.where(oi == _GARBAGE, -1, oi).astype(np.int32)
            out = (ov[:, :max_k], oi[:, :max_k])
    return out, valid, depths, cutoff


def _literal_merge(logits, sv, si, ts, num_bins, m, max_k, dtype):
    """_merge_unconverged_bins_top_k (top_k.py:108-200) as written, on the
    scratch rows ts: tile by tile, with local permutations, range masks and
    the strided packing of slices into 128-lane tiles.  bitonic_topk_arrays
    (an undefined name, :141) is read as bitonic_top_k_arrays: counts
    descending, equal counts in bin order (the network's order is not
    pinned); the final top-128 orders equal values by index.  Reads past the
    row's end (the last tile of an offset) give finfo(dtype).min."""
    vals, idxs = sv[ts].copy(), si[ts].copy()
    bt, vocab = logits.shape
    num_packed_bins = 2 ** O.log2_ceil(-(-max_k // (m - 1)))
    pivot = vals[:, (m - 1) * num_bins:m * num_bins].max(-1, keepdims=True)
    num_gt_k = np.zeros((bt, num_bins), np.int32)
    for i in range(m - 1):
        num_gt_k += (vals[:, i * num_bins:(i + 1) * num_bins] >= pivot).astype(np.int32)
    bin_indices = np.broadcast_to(np.arange(num_bins, dtype=np.int32), (bt, num_bins))
    srt = np.lexsort((bin_indices, -num_gt_k), axis=1)[:, :128]
    sorted_bin_indices = np.take_along_axis(bin_indices, srt, 1)
    packing_perm = np.take_along_axis(sorted_bin_indices,
                                      np.broadcast_to(np.arange(128) % num_packed_bins, (bt, 128)), 1)
    indicator = np.zeros((bt, num_bins), bool)
    for i in range(num_packed_bins):
        indicator |= bin_indices == packing_perm[:, i:i + 1]
    vt = np.int32 if dtype == "i32" else np.float32
    scratch_min = np.iinfo(np.int32).min if dtype == "i32" else np.finfo(np.float32).min   # get_dtype_info(scratch)
    vals = np.concatenate([np.where(indicator, scratch_min, vals[:, i * num_bins:(i + 1) * num_bins])
                           for i in range(vals.shape[1] // num_bins)], axis=1).astype(vt)
    lo = O.dtype_min(dtype)
    packed = [np.full((bt, 128), lo, vt)
              for _ in range(-(-vocab // (128 * (num_bins // num_packed_bins))))]
    xpad = np.full((bt, vocab + 128), lo, vt)
    xpad[:, :vocab] = logits
    lane = np.arange(128)[None, :]
    for offset in range(0, num_bins, 128):
        local_perm = (packing_perm - offset) % 128
        in_range = (packing_perm >= offset) & (packing_perm < offset + 128)
        tiles = [np.take_along_axis(xpad[:, st:st + 128], local_perm, 1) for st in range(offset, vocab, num_bins)]
        for i in range(128 // num_packed_bins):
            pack_mask = (lane >= i * num_packed_bins) & (lane < (i + 1) * num_packed_bins) & in_range
            for j, v in enumerate(tiles[i::128 // num_packed_bins]):
                packed[j] = np.where(pack_mask, v, packed[j])
    packed = np.concatenate(packed, axis=1)
    n = packed.shape[1]
    packed_idxs = (np.arange(n)[None, :] // num_packed_bins) * num_bins + np.concatenate((packing_perm,) * (n // 128), 1)
    val_input = np.concatenate([packed, vals[:, :128]], axis=1)
    idx_input = np.concatenate([packed_idxs, idxs[:, :128]], axis=1)
    order = np.lexsort((idx_input, -val_input.astype(np.float64)), axis=1)[:, :128]
    vals[:, :128] = np.take_along_axis(val_input, order, 1)
    idxs[:, :128] = np.take_along_axis(idx_input, order, 1)
    sv[ts], si[ts] = vals, idxs


def _merge_cases():
    rng = np.random.default_rng(91)
    x = (rng.standard_normal((16, 3000)) * 2).astype(np.float32)
    for r in (5, 6):                       # block 0 cannot converge: 40 spikes in bin 0, 12 in bin 9
        x[r, rng.choice(3000 // 128, 20, replace=False) * 128] = 50.0 + rng.random(20).astype(np.float32)
        x[r, rng.choice(3000 // 128, 12, replace=False) * 128 + 9] = 40.0 + rng.random(12).astype(np.float32)
    k = rng.integers(1, 33, 16).astype(np.int32)
    k[5:7] = 32
    yield "spiked bins, P = 8", "f32", x, k, 32, 8, 128, (3, 6)
    y = np.full((8, 700), -np.inf, np.float32)
    for r in range(8):                     # a few finite values; three spikes share bin 3
        y[r, rng.choice(700, 6 + r, replace=False)] = rng.standard_normal(6 + r).astype(np.float32)
        y[r, [3, 259, 515]] = [9.0, 8.0, 7.0]
    y = O.round_to_dtype(y, "bf16")
    yield "masked bf16 rows past the last slice, P = 16", "bf16", y, np.full(8, 16, np.int32), 16, 4, 256, (2,)
    z = (rng.standard_normal((16, 2000))).astype(np.float32)
    yield "P = num_bins", "f32", z, rng.integers(1, 129, 16).astype(np.int32), 128, 8, 128, (2,)


@pytest.mark.parametrize("replace", [None, -1e12])
@pytest.mark.parametrize("case", list(_merge_cases()), ids=lambda c: c[0] if isinstance(c, tuple) else str(c))
def test_top_dynamic_k_merge_matches_literal_restatement(case, replace):
    """guarantee_convergence=True: the oracle's closed-form packing (column
    (e // P) * num_bins + chosen[e % P]) gives what the tile-level literal
    restatement of _merge_unconverged_bins_top_k gives."""
    _, dt, x, k, max_k, bt, nb, sched = case
    (lv, li), _, _, _ = _literal_dynamic_top_k(x, k, max_k, bt, nb, sched, replace, dt, guarantee_convergence=True)
    ov, oi = O.top_dynamic_k(x, k, max_k, block_token=bt, num_bins=nb, schedule=sched, replace_val=replace,
                             dtype=dt, guarantee_convergence=True)
    assert np.array_equal(oi, li)
    assert np.array_equal(ov.view(np.uint32), lv.view(np.uint32))


def test_top_dynamic_k_merge_reaches_its_paths():
    """The merge cases exercise what they name: unconverged blocks whose
    result the merge changes; outputs that come from packed slots past the
    row's end (index >= cols, value finfo.min); and with P == num_bins every row of an unconverged block gets
    the exact top-k (all bins packed: a closed form)."""
    cases = {c[0]: c for c in _merge_cases()}
    _, dt, x, k, max_k, bt, nb, sched = cases["spiked bins, P = 8"]
    mv, mi = O.top_dynamic_k(x, k, max_k, block_token=bt, num_bins=nb, schedule=sched, guarantee_convergence=True)
    pv, pi, valid, d, _ = O.top_dynamic_k(x, k, max_k, block_token=bt, num_bins=nb, schedule=sched)
    assert not valid and d[5] == max_k and d[6] == max_k
    assert (mi[:8] != pi[:8]).any(axis=1).sum() >= 2 and np.array_equal(mi[8:], pi[8:])
    for r in (5, 6):   # every spike of bin 0, the bin the counts pick, is found; bin 9 keeps its top 6 (m)
        spikes0 = set(np.flatnonzero((x[r] >= 50) & (np.arange(x.shape[1]) % nb == 0)))
        spikes9 = set(np.flatnonzero((x[r] >= 40) & (x[r] < 50)))
        assert len(spikes0) == 20 and spikes0 <= set(mi[r]) and not spikes0 <= set(pi[r])
        assert len(spikes9 & set(mi[r])) == sched[-1]
    _, dt, y, k, max_k, bt, nb, sched = cases["masked bf16 rows past the last slice, P = 16"]
    mv, mi = O.top_dynamic_k(y, k, max_k, block_token=bt, num_bins=nb, schedule=sched, dtype=dt,
                             guarantee_convergence=True)
    past = mi >= y.shape[1]
    assert past.any() and (mv[past] == O.dtype_min(dt)).all()
    _, dt, z, k, max_k, bt, nb, sched = cases["P = num_bins"]
    assert O.packed_bins(max_k, sched[-1]) == nb
    mv, mi = O.top_dynamic_k(z, k, max_k, block_token=bt, num_bins=nb, schedule=sched, guarantee_convergence=True)
    _, _, _, d, _ = O.top_dynamic_k(z, k, max_k, block_token=bt, num_bins=nb, schedule=sched)
    ev, ei = O.top_k(z, max_k)
    unconv = np.repeat((d.reshape(-1, bt) == max_k).any(axis=1), bt)
    assert unconv.sum() >= bt
    assert np.array_equal(mi[unconv], ei[unconv]) and np.array_equal(mv[unconv], ev[unconv])


def test_top_dynamic_k_merge_errors():
    x = np.zeros((8, 300), np.float32)
    with pytest.raises(ValueError):
        O.top_dynamic_k(x, 4, 8, schedule=(1,), guarantee_convergence=True)
    with pytest.raises(NotImplementedError):
        O.top_dynamic_k(x, 4, 8, num_bins=64, schedule=(2,), guarantee_convergence=True)
    O.top_dynamic_k(x, 4, 8, num_bins=64, schedule=(2, 8), guarantee_convergence=True)   # last depth = max_k


def _dyn_cases():
    rng = np.random.default_rng(77)
    # untied values, so that every output (indices included) is pinned
    x = (rng.standard_normal((16, 3000)) * 2).astype(np.float32)
    for r in (5, 6):                       # block 0 cannot converge: 40 spikes in bin 0
        x[r, rng.choice(3000 // 64, 40, replace=False) * 64] = 50.0 + rng.random(40).astype(np.float32)
    k = rng.integers(1, 33, 16).astype(np.int32)
    yield "unconverged block, depth_upper > m_final", x, k, 32, 8, 64, (3, 6, 12)
    yield "early exit per block", x, np.full(16, 4, np.int32), 32, 4, 64, (2, 3, 6, 12)
    y = (rng.standard_normal((8, 700)) * 3).astype(np.float32)
    y[:, ::7] = -np.inf
    yield "short rows, fillers", y, rng.integers(1, 17, 8).astype(np.int32), 16, 4, 32, (2, 5)
    z = (rng.standard_normal((8, 4000))).astype(np.float32)
    yield "k = max_k everywhere", z, np.full(8, 24, np.int32), 24, 8, 128, (2, 4, 7)


@pytest.mark.parametrize("replace", [None, -1e12])
@pytest.mark.parametrize("case", list(_dyn_cases()), ids=lambda c: c[0] if isinstance(c, tuple) else str(c))
def test_top_dynamic_k_matches_literal_block_restatement(case, replace):
    """All five outputs of O.top_dynamic_k equal the literal block-by-block
    restatement of dynamic_top_k_refs, including blocks that stop early, rows
    that never converge (depth max_k, valid False) and depth_upper buckets
    past the last step (ranks never written keep finfo.min)."""
    _, x, k, max_k, bt, nb, sched = case
    (lv, li), lvalid, ld, lc = _literal_dynamic_top_k(x, k, max_k, bt, nb, sched, replace)
    ov, oi, ovalid, od, oc = O.top_dynamic_k(x, k, max_k, block_token=bt, num_bins=nb, schedule=sched,
                                             replace_val=replace)
    assert ovalid == lvalid
    assert np.array_equal(od, ld) and np.array_equal(oc.view(np.uint32), lc.view(np.uint32))
    assert np.array_equal(oi, li)
    assert np.array_equal(ov.view(np.uint32), lv.view(np.uint32))


def _full_depth_variant(x, k, max_k, block_token, num_bins, schedule, replace_val, depths):
    """The same selection with every rank of the depth_upper bucket filled
    (what a scan to full depth gives): what the oracle did before it kept
    never-evaluated ranks at finfo.min."""
    sch = O.topm_schedule(max_k, num_bins, block_token, schedule)
    gts = sorted(set(2 ** O.log2_ceil(s - 1) if s > 1 else s for s in sch))
    gmax, up = int(depths.max()), gts[-1]
    for a, b in zip(gts, gts[1:]):
        if a < gmax <= b:
            up = b
            break
    fv, fi = O.binned_topm(x, up, num_bins)
    sv, si = fv.reshape(len(x), -1), fi.reshape(len(x), -1)
    order = np.lexsort((np.where(si < 0, 2 ** 40, si), -np.where(si < 0, -np.inf, sv.astype(np.float64))), axis=1)
    gv = np.take_along_axis(sv, order[:, :max_k], 1)
    gi = np.take_along_axis(si, order[:, :max_k], 1)
    if replace_val is not None:
        gv = np.where(np.arange(max_k)[None, :] < np.asarray(k)[:, None], gv, np.float32(replace_val))
    return gv.astype(np.float32), gi


def test_literal_restatement_reaches_the_unconverged_paths():
    """The cases above really exercise what they name: a block that never
    converges (depth max_k, valid False) and blocks that stop before the
    depth_upper bucket, where the never-written ranks change the result
    against a full-depth scan: indices with replace_val=None, and values inside
    the first k[row] positions of an unconverged row with replace_val set."""
    cases = {c[0]: c for c in _dyn_cases()}
    _, x, k, max_k, bt, nb, sched = cases["unconverged block, depth_upper > m_final"]
    for rep in (None, -1e12):
        (lv, li), valid, d, _ = _literal_dynamic_top_k(x, k, max_k, bt, nb, sched, rep)
        assert not valid and d[5] == max_k and (d[8:] < max_k).all()
        fv, fi = _full_depth_variant(x, k, max_k, bt, nb, sched, rep, d)
        assert (fv.view(np.uint32) != lv.view(np.uint32)).any(axis=1).sum() >= 1
    _, x, k, max_k, bt, nb, sched = cases["early exit per block"]
    (lv, li), valid, d, c = _literal_dynamic_top_k(x, k, max_k, bt, nb, sched)
    assert valid and (d == 1).sum() >= 8
    fv, fi = _full_depth_variant(x, k, max_k, bt, nb, sched, None, d)
    assert (fi != li).any(axis=1).sum() >= 4
