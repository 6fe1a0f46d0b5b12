"""GPU parity: exact top-k, the fused sampler and top_p_and_sample through the
C ABI, against the oracle on identical seeded inputs (bit-exact values,
indices and token ids)."""
import numpy as np
import pytest
import torch

from oracle import tallax_oracle as O
from tests.gpu_util import bits, from_dev_vals, host_values, to_dev

pytestmark = pytest.mark.gpu


def _log(msg):
    print(msg, flush=True)


# --------------------------------------------------------------------------- primitives
def test_lane_exchange_semantics(gpu):
    """DPP / v_permlane*_swap lane exchanges used by every wave network."""
    from tallax_amd import _lib
    out = torch.zeros(7 * 64, dtype=torch.int32, device=gpu)
    _lib.check(_lib.LIB.tallax_testing_lane_ops(out.data_ptr(), _lib.stream_of(out)), "lane_ops")
    torch.cuda.synchronize()
    o = out.cpu().numpy().reshape(7, 64)
    lanes = np.arange(64)
    for d in range(6):
        assert np.array_equal(o[d], lanes ^ (1 << d)), d
    assert np.array_equal(o[6], 63 - lanes)


def test_exp_log_bitexact(gpu):
    from tallax_amd import _lib
    rng = np.random.default_rng(11)
    x = np.concatenate([
        rng.uniform(-110, 95, 200000), rng.uniform(-1, 1, 50000),
        rng.integers(0, 0x7F800000, 100000).astype(np.uint32).view(np.float32).astype(np.float64),
        [0.0, -0.0, 1.0, np.inf, -np.inf, np.nan, -1.0, 1e-45, 88.72, -103.97, 2.0**-126]]).astype(np.float32)
    xd = torch.from_numpy(x).to(gpu)
    e = torch.empty_like(xd); l = torch.empty_like(xd)
    _lib.check(_lib.LIB.tallax_testing_expf_logf(xd.data_ptr(), e.data_ptr(), l.data_ptr(), x.size,
                                                 _lib.stream_of(xd)), "expf_logf")
    torch.cuda.synchronize()
    ge, gl = e.cpu().numpy(), l.cpu().numpy()
    oe, ol = O.exp_f32(x), O.log_f32(x)
    nan_e = np.isnan(oe); nan_l = np.isnan(ol)
    assert np.array_equal(np.isnan(ge), nan_e) and np.array_equal(np.isnan(gl), nan_l)
    assert np.array_equal(bits(ge)[~nan_e], bits(oe)[~nan_e])
    assert np.array_equal(bits(gl)[~nan_l], bits(ol)[~nan_l])


def test_gumbel_bitexact(gpu):
    from tallax_amd import _lib
    rng = np.random.default_rng(12)
    ctr = rng.integers(0, 2**32, 300000, dtype=np.uint64).astype(np.uint32)
    cd = torch.from_numpy(ctr.view(np.int32)).to(gpu)
    g = torch.empty(ctr.size, dtype=torch.float32, device=gpu)
    b = torch.empty(ctr.size, dtype=torch.int32, device=gpu)
    _lib.check(_lib.LIB.tallax_testing_gumbel(0x12345678, 0x9abcdef0, cd.data_ptr(), g.data_ptr(),
                                              b.data_ptr(), ctr.size, _lib.stream_of(cd)), "gumbel")
    torch.cuda.synchronize()
    o0, o1 = O.threefry2x32(0x12345678, 0x9abcdef0, np.zeros_like(ctr), ctr)
    assert np.array_equal(b.cpu().numpy().view(np.uint32), o0 ^ o1)
    og = -O.log_f32(-O.log_f32(O.sparse_random_uniform((0x12345678, 0x9abcdef0), (np.zeros(ctr.size, np.int64), ctr.astype(np.int64)), 1, minval=O.TINY)))
    # counter here is 0 * 1 + ctr
    assert np.array_equal(bits(g.cpu().numpy()), bits(og))


# --------------------------------------------------------------------------- top-k
TOPK_CASES = [
    # rows, cols, k, dtype, kind
    (8, 32768, 64, "f32", "normal"),        # config 1
    (13, 167, 5, "f32", "normal"),          # ragged, misaligned rows
    (3, 1000, 100, "bf16", "normal"),
    (16, 4097, 64, "f32", "ints"),          # heavy ties
    (4, 128, 128, "f32", "normal"),         # k == cols
    (5, 300, 128, "bf16", "ints"),
    (2, 5000, 17, "f32", "const"),          # every value equal: exact bisection path
    (6, 20000, 50, "f32", "special"),       # NaN / -inf / -0 / finfo.min
    (7, 70001, 128, "bf16", "normal"),      # odd length bf16 (misaligned rows)
    (32, 201088, 64, "bf16", "normal"),     # the reference's own top-k benchmark shape
    (4, 131072, 128, "bf16", "sorted_asc"), # structured inputs: weak thread-maxima bound
    (4, 131072, 50, "f32", "sorted_desc"),
    (8, 65536, 100, "bf16", "strided_hot"), # one thread owns a candidate in every vector
    (8, 65536, 100, "f32", "strided_hot"),
    (16, 128256, 128, "bf16", "normal"),    # vocabulary row of config 4
    # heavy ties: the exact tie selection (k-th key by bisection, then the
    # first elements of that key in slot order)
    (256, 128256, 128, "bf16", "const"),    # constant rows at config 4's shape (whole-row workgroups)
    (64, 128256, 128, "bf16", "masked5"),   # -inf but 5 values per row (constrained decoding)
    (8, 151936, 50, "f32", "masked5"),      # the same, segmented rows
    (4, 40000, 100, "bf16", "tieblock"),    # 60 large values, then a 10000-wide tie block
    (4, 40000, 100, "f32", "tieblock"),
    (4, 40000, 100, "f32", "nan_heavy"),    # NaN rows with a few finite, -inf and finfo.min values
    # the same inputs on rows too long for one workgroup that do not divide
    # into whole-row parts (segments, then the merge)
    (2, 200003, 17, "f32", "const"),
    (3, 200003, 64, "f32", "ints"),
    (6, 200003, 50, "f32", "special"),
    (4, 200003, 100, "bf16", "tieblock"),
    (4, 200003, 100, "f32", "tieblock"),
    (4, 200003, 100, "f32", "nan_heavy"),
    # ... and rows that do: 2-4 whole-row parts, then the merge (misaligned
    # parts when a part is not a whole number of vectors)
    (8, 200000, 64, "f32", "normal"),
    (4, 151938, 100, "f32", "special"),
    (4, 200000, 100, "bf16", "tieblock"),
    (2, 200000, 17, "f32", "const"),
    (16, 151936, 128, "f32", "masked5"),
    (32, 151936, 128, "f32", "masked_mix"),
    # whole rows at 19 vectors per thread (bf16 rows up to 155648 elements,
    # f32 up to 77824), aligned and misaligned, with the rare paths
    (128, 151936, 50, "bf16", "normal"),
    (6, 151931, 50, "bf16", "special"),
    (16, 151936, 128, "bf16", "const"),
    (8, 151936, 100, "bf16", "tieblock"),
    (64, 151936, 128, "bf16", "masked5"),
    (96, 151936, 128, "bf16", "masked_mix"),
    (8, 70001, 64, "f32", "normal"),
    (4, 77000, 100, "f32", "nan_heavy"),
    # whole-row workgroups on masked rows: fewer than 128 eligible values take
    # the rest of the list by class (finfo.min, -inf, NaN, each in index order)
    (256, 128256, 128, "bf16", "masked_mix"),
    (128, 32768, 100, "f32", "masked_mix"),
    (160, 5003, 128, "bf16", "masked_mix"),
    (128, 100, 64, "f32", "masked_mix"),    # rows shorter than 128
    # whole-row workgroups: the bound from the first half of every thread's
    # vectors (positive rows), the whole-row bound (negative rows), overflow
    # from the first path into the exact tie selection, and misaligned rows
    # where thread 0 owns both the row's first and its last vector
    (256, 128256, 128, "bf16", "normal"),
    (128, 65536, 100, "f32", "normal"),
    (128, 65536, 100, "bf16", "negative"),
    (128, 65536, 64, "bf16", "tieblock"),
    (128, 8195, 128, "bf16", "normal"),
    (128, 4097, 64, "f32", "normal"),
]


def _masked_mix(rows, cols, rng):
    """Rows of -inf with a few allowed values: row r % 8 == 0 allows none,
    1-3 allow 1..127, 4-5 a few hundred; rows 6 mix finfo.min and NaN in
    (all ineligible classes, sparse and out of order); rows 7 are unmasked."""
    x = np.full((rows, cols), -np.inf, np.float32)
    fmin = np.finfo(np.float32).min
    for r in range(rows):
        kind = r % 8
        if kind == 7:
            x[r] = rng.standard_normal(cols)
            continue
        n = 0 if kind == 0 else (rng.integers(1, 128) if kind <= 3 else rng.integers(128, 600))
        if kind == 6:
            n = rng.integers(0, 100)
            spots = rng.choice(cols, min(cols, 300), replace=False)
            x[r, spots[: len(spots) // 3]] = fmin
            x[r, spots[len(spots) // 3: 2 * len(spots) // 3]] = np.nan
        n = min(n, cols)
        x[r, rng.choice(cols, n, replace=False)] = (rng.standard_normal(n) * 3).astype(np.float32)
    return x


def _make(rows, cols, kind, seed):
    rng = np.random.default_rng(seed)
    if kind == "sorted_asc":
        return np.sort(rng.standard_normal((rows, cols)).astype(np.float32), axis=1)
    if kind == "sorted_desc":
        return -np.sort(rng.standard_normal((rows, cols)).astype(np.float32), axis=1)
    if kind == "strided_hot":
        # elements (j * 256 + 5) * vec for j = 0..63 are large: with 256 threads
        # per workgroup and vec elements per 16-byte vector they all fall to one thread
        x = rng.standard_normal((rows, cols)).astype(np.float32)
        for vec in (4, 8):
            idx = (np.arange(64) * 256 + 5) * vec
            idx = idx[idx < cols]
            x[:, idx] = 20.0 + np.arange(idx.size, dtype=np.float32) / 8
        return x
    if kind == "normal":
        return rng.standard_normal((rows, cols)).astype(np.float32)
    if kind == "negative":
        return (rng.standard_normal((rows, cols)) - 20).astype(np.float32)
    if kind == "ints":
        return rng.integers(-6, 7, (rows, cols)).astype(np.float32)
    if kind == "const":
        return np.full((rows, cols), 1.5, np.float32)
    if kind == "masked5":
        x = np.full((rows, cols), -np.inf, np.float32)
        for r in range(rows):
            x[r, rng.choice(cols, 5, replace=False)] = rng.standard_normal(5).astype(np.float32)
        return x
    if kind == "tieblock":
        x = (rng.standard_normal((rows, cols)) * 0.1 - 10).astype(np.float32)
        for r in range(rows):
            pos = rng.choice(cols, 10060, replace=False)
            x[r, pos[:60]] = 100 + rng.random(60).astype(np.float32) * 50
            x[r, pos[60:]] = 5.0
        return x
    if kind == "masked_mix":
        return _masked_mix(rows, cols, rng)
    if kind == "nan_heavy":
        x = np.full((rows, cols), np.nan, np.float32)
        for r in range(rows):
            pos = rng.choice(cols, 90, replace=False)
            x[r, pos[:50]] = rng.standard_normal(50).astype(np.float32)
            x[r, pos[50:70]] = -np.inf
            x[r, pos[70:]] = np.finfo(np.float32).min
        return x
    x = rng.standard_normal((rows, cols)).astype(np.float32)
    u = rng.random((rows, cols))
    x[u < 0.05] = np.nan
    x[(u >= 0.05) & (u < 0.1)] = -np.inf
    x[(u >= 0.1) & (u < 0.2)] = -0.0
    x[(u >= 0.2) & (u < 0.22)] = np.finfo(np.float32).min
    x[0, :] = np.nan   # a row with no eligible value at all
    x[1, : cols // 2] = 0.0
    return x


@pytest.mark.parametrize("rows,cols,k,dtype,kind", TOPK_CASES)
def test_topk_parity(gpu, rows, cols, k, dtype, kind):
    from tallax_amd import tax
    _log(f"top_k rows={rows} cols={cols} k={k} dtype={dtype} kind={kind}")
    x = _make(rows, cols, kind, seed=rows * 7919 + cols)
    xv = host_values(x, dtype)
    vals, idx = tax.top_k(to_dev(x, dtype, gpu), k)
    torch.cuda.synchronize()
    ov, oi = O.top_k(xv, k, dtype)
    gi = idx.cpu().numpy()
    gv = from_dev_vals(vals)
    assert np.array_equal(gi, oi)
    assert np.array_equal(bits(gv), bits(ov))


@pytest.mark.parametrize("rows,cols,k", [(1000, 1, 1), (1000, 7, 3), (5000, 16, 16), (3000, 17, 2), (5000, 32, 8),
                                         (3000, 33, 5), (2000, 64, 64), (2000, 100, 8), (700, 128, 128),
                                         (700, 129, 1), (500, 256, 100), (66000, 64, 2), (3000, 257, 8),
                                         (2000, 512, 128), (1000, 513, 50), (999, 1024, 64), (8192, 1500, 7),
                                         (300, 2048, 128)])
@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_topk_short_rows(gpu, rows, cols, k, dtype):
    """Short rows (one thread, one wave or one small block per row, by length and row count): heavy
    ties, signed zeros, NaNs, +-inf and finfo.min, against the oracle."""
    from tallax_amd import tax
    _log(f"top_k short rows={rows} cols={cols} k={k} {dtype}")
    rng = np.random.default_rng(rows * 31 + cols + k)
    x = np.round(rng.standard_normal((rows, cols)) * 2).astype(np.float32) / 2
    fmin = np.float32(-3.3895314e38) if dtype == "bf16" else np.finfo(np.float32).min
    special = np.array([np.nan, -0.0, 0.0, np.inf, -np.inf, fmin, -np.nan], np.float32)
    mask = rng.random((rows, cols)) < 0.15
    x[mask] = rng.choice(special, int(mask.sum()))
    x[::11] = np.nan                      # rows with nothing admissible
    xv = host_values(x, dtype)
    vals, idx = tax.top_k(to_dev(x, dtype, gpu), k)
    torch.cuda.synchronize()
    ov, oi = O.top_k(xv, k, dtype)
    assert np.array_equal(idx.cpu().numpy(), oi)
    assert np.array_equal(bits(from_dev_vals(vals)), bits(ov))


@pytest.mark.parametrize("rows,cols,k", [(70000, 300, 8), (66000, 1024, 64)])
def test_topk_more_rows_than_a_grid_dimension(gpu, rows, cols, k):
    """More than 65535 rows: every launch is a one-dimensional grid."""
    from tallax_amd import tax
    _log(f"top_k rows={rows} cols={cols} k={k}")
    rng = np.random.default_rng(rows + k)
    x = np.round(rng.standard_normal((rows, cols)) * 16).astype(np.float32) / 16
    vals, idx = tax.top_k(torch.from_numpy(x).to(gpu), k)
    torch.cuda.synchronize()
    ov, oi = O.top_k(x, k)
    assert np.array_equal(idx.cpu().numpy(), oi)
    assert np.array_equal(bits(vals.cpu().numpy()), bits(ov))


def test_topk_config3_spikes(gpu):
    """Config 3: f32 [128, 151936], N(0, sigma=2) plus 32 spikes per row at
    exactly 8.0 (32-way ties inside the top-50), k=50."""
    from tallax_amd import tax
    rng = np.random.default_rng(3)
    x = (rng.standard_normal((128, 151936)) * 2).astype(np.float32)
    for r in range(128):
        x[r, rng.choice(151936, 32, replace=False)] = 8.0
    vals, idx = tax.top_k(to_dev(x, "f32", gpu), 50)
    torch.cuda.synchronize()
    ov, oi = O.top_k(x, 50)
    assert np.array_equal(idx.cpu().numpy(), oi)
    assert np.array_equal(bits(vals.cpu().numpy()), bits(ov))


@pytest.mark.parametrize("rows,cols,k,dtype", [(256, 128256, 128, "bf16"), (128, 151936, 50, "f32"),
                                               (16, 5003, 77, "bf16"), (3000, 12, 5, "f32"), (2000, 40, 8, "bf16"),
                                               (700, 256, 100, "f32")])   # short rows: one thread / wave per row
def test_topk_replace_per_row_k(gpu, rows, cols, k, dtype):
    """tallax_topk_replace through the C ABI: the exact top-k whose positions
    >= k_rows[row] hold replace_val rounded to the input dtype
    (top_k.py:365-369 on a converged run)."""
    from tallax_amd import _lib
    _log(f"topk_replace rows={rows} cols={cols} k={k} dtype={dtype}")
    rng = np.random.default_rng(rows + cols)
    x = (rng.standard_normal((rows, cols)) * 3).astype(np.float32)
    kr = rng.integers(0, k + 1, rows).astype(np.int32)
    xd = to_dev(x, dtype, gpu)
    krd = torch.from_numpy(kr).to(gpu)
    vals = torch.empty((rows, k), dtype=xd.dtype, device=gpu)
    idx = torch.empty((rows, k), dtype=torch.int32, device=gpu)
    dt = _lib.dtype_code(xd)
    need = _lib.LIB.tallax_topk_workspace_size(rows, cols, k, dt)
    ws = torch.empty(max(need, 1), dtype=torch.uint8, device=gpu)
    _lib.check(_lib.LIB.tallax_topk_replace(xd.data_ptr(), dt, rows, cols, k, krd.data_ptr(), -1e12,
                                            vals.data_ptr(), idx.data_ptr(), ws.data_ptr(), ws.numel(),
                                            _lib.stream_of(xd)), "topk_replace")
    torch.cuda.synchronize()
    ov, oi = O.top_k(host_values(x, dtype), k, dtype)
    ov = np.where(np.arange(k)[None, :] < kr[:, None], ov, O.round_to_dtype(np.float32(-1e12), dtype))
    assert np.array_equal(idx.cpu().numpy(), oi)
    assert np.array_equal(bits(from_dev_vals(vals)), bits(ov))


def test_topk_repeated_calls_reuse_workspace(gpu):
    from tallax_amd import tax
    rng = np.random.default_rng(5)
    for i, (rows, cols) in enumerate([(64, 50000), (8, 100000), (64, 50000)]):
        x = rng.standard_normal((rows, cols)).astype(np.float32)
        v, ix = tax.top_k(to_dev(x, "f32", gpu), 128)
        torch.cuda.synchronize()
        assert np.array_equal(ix.cpu().numpy(), O.top_k(x, 128)[1]), i


# --------------------------------------------------------------------------- sampler
def _sampler_inputs(rows, vocab, seed, sigma=3.0):
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal((rows, vocab)) * sigma).astype(np.float32)
    temp = rng.uniform(0.5, 1.5, rows).astype(np.float32)
    topk = rng.integers(1, 1025, rows).astype(np.int32)
    topp = rng.uniform(0.7, 1.0, rows).astype(np.float32)
    return x, temp, topk, topp


@pytest.mark.parametrize("rows,vocab,dtype,masked", [(256, 128256, "bf16", False), (64, 32000, "f32", False),
                                                     (16, 4096, "bf16", False), (8, 131, "f32", False),
                                                     (256, 128256, "bf16", True), (128, 32768, "f32", True),
                                                     (128, 8195, "bf16", False), (64, 151936, "bf16", False),
                                                     (32, 151936, "bf16", True), (8, 70001, "f32", False),
                                                     (16, 200003, "bf16", False), (32, 151936, "f32", False),
                                                     (16, 201088, "f32", True), (32, 256000, "bf16", False)])
def test_fused_sampler_parity(gpu, rows, vocab, dtype, masked):
    from tallax_amd import sampling
    _log(f"sample rows={rows} vocab={vocab} dtype={dtype} masked={masked}")
    x, temp, topk, topp = _sampler_inputs(rows, vocab, seed=vocab + rows)
    if masked:   # constrained decoding: most logits -inf
        x = _masked_mix(rows, vocab, np.random.default_rng(rows))
    temp[::17] = 1e-6      # greedy rows
    topk[1::13] = 1        # top-1 rows
    topp[2::11] = 0.9999999
    key = (0, 1234)
    meta = sampling.SamplingMetadata(torch.from_numpy(topk), torch.from_numpy(topp), torch.from_numpy(temp))
    tok = sampling.sample(key, to_dev(x, dtype, gpu), meta)
    torch.cuda.synchronize()
    want = O.sample(key, host_values(x, dtype), topk, topp, temp, dtype=dtype)
    assert np.array_equal(tok.cpu().numpy(), want)


def test_fused_sampler_dim0_offset_and_key(gpu):
    from tallax_amd import sampling
    x, temp, topk, topp = _sampler_inputs(32, 50000, seed=9)
    meta = sampling.SamplingMetadata(torch.from_numpy(topk), torch.from_numpy(topp), torch.from_numpy(temp))
    for key, off in [((0, 7), 0), ((0xDEADBEEF, 0x01234567), 96)]:
        tok = sampling.sample(key, to_dev(x, "f32", gpu), meta, dim0_offset=off)
        torch.cuda.synchronize()
        want = O.sample(key, x, topk, topp, temp, dtype="f32", dim0_offset=off)
        assert np.array_equal(tok.cpu().numpy(), want)


@pytest.mark.parametrize("k,dtype", [(128, "f32"), (128, "bf16"), (64, "f32"), (50, "f32"), (8, "bf16"), (1, "f32")])
def test_top_p_and_sample_parity(gpu, k, dtype):
    from tallax_amd import sampling
    rng = np.random.default_rng(100 + k)
    B = 300
    L = -np.sort(-(rng.standard_normal((B, k)) * 2).astype(np.float32), axis=1)
    L = host_values(L, dtype)
    L = -np.sort(-L, axis=1)
    I = rng.integers(0, 50000, (B, k)).astype(np.int32)
    tp = rng.uniform(0.5, 1.0, B).astype(np.float32)
    tt = rng.uniform(0.3, 2.0, B).astype(np.float32)
    key = (3, 4)
    tok = sampling.top_p_and_sample(to_dev(L, dtype, gpu), torch.from_numpy(I).to(gpu), key,
                                    torch.from_numpy(tp), torch.from_numpy(tt), vocab_size=50000,
                                    replace_val=-1e12)
    torch.cuda.synchronize()
    want = O.top_p_and_sample(L, I, key, tp, tt, 50000, -1e12)
    assert np.array_equal(tok.cpu().numpy(), want)


@pytest.mark.parametrize("k", [128, 100, 64, 9, 1])
def test_top_p_mask_parity(gpu, k):
    """sampling.top_p_mask (sampling.py:25-62, axis 0) against the oracle, bit
    for bit: random columns, ties at the threshold, p = 1 (t may reach k: the
    out-of-range gather keeps everything >= 0.0), tiny p (only the maximum and
    its ties survive), and a constant column."""
    from tallax_amd import sampling
    rng = np.random.default_rng(500 + k)
    B = 257
    L = -np.sort(-(np.round(rng.standard_normal((k, B)) * 4) / 4).astype(np.float32), axis=0)
    L[:, 1] = 0.75  # constant column
    p = rng.uniform(0.3, 1.0, B).astype(np.float32)
    p[2], p[3], p[4] = 1.0, np.float32(1e-7), 0.0
    got = sampling.top_p_mask(topk_logits=torch.from_numpy(L).to(gpu), p=torch.from_numpy(p), replace_val=-1e12,
                              axis=0)
    torch.cuda.synchronize()
    want = O.top_p_mask(L, p, -1e12)
    assert got.dtype == torch.float32 and tuple(got.shape) == (k, B)
    assert np.array_equal(got.cpu().numpy().view(np.uint32), want.view(np.uint32))
    # scalar p broadcasts over the columns
    got2 = sampling.top_p_mask(topk_logits=torch.from_numpy(L).to(gpu), p=0.9, replace_val=-5.0, axis=0)
    torch.cuda.synchronize()
    want2 = O.top_p_mask(L, np.full(B, 0.9, np.float32), -5.0)
    assert np.array_equal(got2.cpu().numpy().view(np.uint32), want2.view(np.uint32))


def test_top_p_mask_errors(gpu):
    from tallax_amd import sampling
    x = torch.zeros((8, 4), device=gpu)
    with pytest.raises(NotImplementedError):
        sampling.top_p_mask(topk_logits=x, p=0.9, replace_val=0.0, axis=1)
    with pytest.raises(NotImplementedError):
        sampling.top_p_mask(topk_logits=torch.zeros((129, 4), device=gpu), p=0.9, replace_val=0.0, axis=0)
    with pytest.raises(NotImplementedError):
        sampling.top_p_mask(topk_logits=x.to(torch.bfloat16), p=0.9, replace_val=0.0, axis=0)


@pytest.mark.parametrize("rows,vocab,dtype,widths", [
    (256, 128256, "bf16", [128256 // 8] * 8),           # 8-way vocab split of config 4: [256, 16032] shards
    (256, 128256, "bf16", [64128, 64128]),
    (64, 50000, "f32", [20000, 129, 29871]),            # uneven, a shard barely over 128 columns
    (32, 32000, "bf16", [32000]),
    (16, 400000, "f32", [200000, 200000]),              # shards of 4 whole-row parts each (offsets composed)
    (8, 400006, "f32", [200003, 200003]),               # shards of segments
])
def test_sample_sharded_equals_sample(gpu, rows, vocab, dtype, widths):
    """The vocabulary-sharded composition (per-shard top-128, global indices,
    concatenation, top-128 merge, k mask, tail: sampling.py:300-321) gives the
    tokens of the unsharded sampler and of the oracle."""
    from tallax_amd import sampling
    assert sum(widths) == vocab
    x, temp, topk, topp = _sampler_inputs(rows, vocab, seed=rows + len(widths))
    x[1, :] = 0.5                          # a constant row: ties across shards go to the lowest index
    x[2, ::1000] = 9.0                     # equal maxima in several shards
    temp[::13] = 1e-6                      # greedy rows
    meta = sampling.SamplingMetadata(torch.from_numpy(topk), torch.from_numpy(topp), torch.from_numpy(temp))
    full = to_dev(x, dtype, gpu)
    bounds = np.cumsum([0] + widths)
    shards = [full[:, bounds[i]:bounds[i + 1]].contiguous() for i in range(len(widths))]
    key = torch.tensor([7, 99], dtype=torch.int32, device=gpu)
    got = sampling.sample_sharded(key, shards, meta, dim0_offset=5)
    want = sampling.sample(key, full, meta, dim0_offset=5)
    torch.cuda.synchronize()
    assert np.array_equal(got.cpu().numpy(), want.cpu().numpy())
    ref = O.sample((7, 99), host_values(x, dtype), topk, topp, temp, dtype=dtype, dim0_offset=5)
    assert np.array_equal(got.cpu().numpy(), ref)
