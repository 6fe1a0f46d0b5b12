"""GPU parity on the reference's own test matrices, case for case, against the
oracle (bit-exact) rather than the reference's acceptance predicates:

  * tests/sort_test.py:15-61        dtype x size x variant x (arrays, keys) on (16, size)
  * tests/take_along_axis_test.py   num_tokens x vocab x k x axis, and (8, 2048) k=1024
  * tests/cumsum_test.py:10-33      shape x axis x dtype x reverse
  * tests/tumpy_sort_test.py        every test of the file
  * tests/bitonic_topk_test.py      top-k (k = min(128, cols)) and top-1 along both
                                    axes, float32 and int32 (randint(0, 1000))

The reference draws its inputs from jax.random, which is not installed here;
the same shapes and distributions come from seeded numpy generators, and the
oracle sees the very arrays the GPU does."""
import numpy as np
import pytest
import torch

from oracle import tallax_oracle as O
from tests.gpu_util import bits, from_dev_vals, to_dev

pytestmark = pytest.mark.gpu


def _log(msg):
    print(msg, flush=True)


def _host(t: torch.Tensor) -> np.ndarray:
    return from_dev_vals(t) if t.dtype == torch.bfloat16 else t.cpu().numpy()


def _same(a: np.ndarray, b: np.ndarray) -> bool:
    if a.dtype == np.int32 or b.dtype == np.int32:
        return np.array_equal(a, b)
    return np.array_equal(bits(a), bits(b))


# --------------------------------------------------------------------------- sort_test.py:15-61
@pytest.mark.parametrize("num_arrays,num_keys", [(1, 1), (2, 1), (2, 2)])
@pytest.mark.parametrize("variant", ["standard", "return_argsort", "return_argsort_stable", "descending",
                                     "descending_argsort", "descending_stable"])
@pytest.mark.parametrize("size", [128, 256, 2048, 131072])
@pytest.mark.parametrize("dtype", ["bf16", "f32"])
def test_sort_comprehensive(gpu, dtype, size, variant, num_arrays, num_keys):
    from tallax_amd import tax
    return_argsort = "return_argsort" in variant   # as written: "descending_argsort" does not ask for it
    is_stable = "stable" in variant
    descending = "descending" in variant
    _log(f"sort_test {dtype} (16, {size}) {variant} arrays={num_arrays} keys={num_keys}")
    rng = np.random.default_rng(size * 7 + num_arrays * 3 + num_keys)
    host, dev = [], []
    for _ in range(num_arrays):
        x = rng.standard_normal((16, size)).astype(np.float32)
        host.append(O.round_to_dtype(x, dtype))
        dev.append(to_dev(x, dtype, gpu))
    got = tax.sort(dev, num_keys=num_keys, is_stable=is_stable, return_argsort=return_argsort,
                   descending=descending)
    torch.cuda.synchronize()
    want, _ = O.sort(host, num_keys, is_stable=is_stable, return_argsort=return_argsort, descending=descending,
                     dtypes=[dtype] * num_arrays)
    assert len(got) == len(want)
    for g, w in zip(got, want):
        assert _same(_host(g), w)


# --------------------------------------------------------------------------- take_along_axis_test.py
@pytest.mark.parametrize("axis", [0, 1])
@pytest.mark.parametrize("k", [64, 128, 200, 300])
@pytest.mark.parametrize("vocab_size", [128, 256, 300])
@pytest.mark.parametrize("num_tokens", [8, 16, 13])
def test_take_along_axis(gpu, num_tokens, vocab_size, k, axis):
    from tallax_amd import tumpy
    _log(f"take_along_axis_test tokens={num_tokens} vocab={vocab_size} k={k} axis={axis}")
    rng = np.random.default_rng(num_tokens * 1000 + vocab_size * 10 + k + axis)
    if axis == 1:
        values = rng.standard_normal((num_tokens, vocab_size)).astype(np.float32)
        indices = rng.integers(0, vocab_size, (num_tokens, k)).astype(np.int32)
    else:
        values = rng.standard_normal((vocab_size, num_tokens)).astype(np.float32)
        indices = rng.integers(0, vocab_size, (k, num_tokens)).astype(np.int32)
    got = tumpy.take_along_axis(torch.from_numpy(values).to(gpu), torch.from_numpy(indices).to(gpu), axis)
    torch.cuda.synchronize()
    want = np.take_along_axis(values, indices, axis=axis)
    assert np.array_equal(bits(got.cpu().numpy()), bits(want))
    assert np.array_equal(bits(want), bits(O.take_along_axis(values, indices, axis)))


def test_take_along_axis_large_k(gpu):
    from tallax_amd import tumpy
    rng = np.random.default_rng(1)
    values = rng.standard_normal((8, 2048)).astype(np.float32)
    indices = rng.integers(0, 2048, (8, 1024)).astype(np.int32)
    got = tumpy.take_along_axis(torch.from_numpy(values).to(gpu), torch.from_numpy(indices).to(gpu), 1)
    torch.cuda.synchronize()
    assert np.array_equal(bits(got.cpu().numpy()), bits(np.take_along_axis(values, indices, 1)))


# --------------------------------------------------------------------------- cumsum_test.py:10-33
@pytest.mark.parametrize("reverse", [False, True])
@pytest.mark.parametrize("dtype", ["f32", "i32"])
@pytest.mark.parametrize("axis", [0, 1])
@pytest.mark.parametrize("shape", [(8, 128), (16, 256), (128, 8), (256, 16), (13, 167)])
def test_cumsum_correctness(gpu, shape, axis, dtype, reverse):
    """float32: bit-exact against the oracle's restatement of the reference's
    summation order (cumsum.py:16-63), and within the reference test's own
    tolerance (rtol 1e-3, atol 1e-6) of the float64 scan; int32: exact."""
    from tallax_amd import tax
    _log(f"cumsum_test {shape} axis={axis} {dtype} reverse={reverse}")
    rng = np.random.default_rng(42 + shape[0] + shape[1] + axis)
    if dtype == "f32":
        x = rng.standard_normal(shape).astype(np.float32)
    else:
        x = rng.integers(0, 100, shape).astype(np.int32)
    got = tax.cumsum(torch.from_numpy(x).to(gpu), axis=axis, reverse=reverse).cpu().numpy()
    flip = (lambda a: np.flip(a, axis)) if reverse else (lambda a: a)
    if dtype == "f32":
        assert np.array_equal(bits(got), bits(O.cumsum(x, axis, reverse)))
        ref64 = flip(np.cumsum(flip(x.astype(np.float64)), axis=axis))
        np.testing.assert_allclose(got, ref64, rtol=1e-3, atol=1e-6)
    else:
        assert got.dtype == np.int32
        assert np.array_equal(got, flip(np.cumsum(flip(x), axis=axis)).astype(np.int32))


# --------------------------------------------------------------------------- tumpy_sort_test.py
def _dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to("cuda")


def test_tumpy_sort(gpu):
    from tallax_amd import tumpy as tnp
    a = np.random.default_rng(0).integers(0, 100, (2, 16)).astype(np.int32)
    assert np.array_equal(tnp.sort(_dev(a), axis=-1).cpu().numpy(), np.sort(a, axis=-1))


def test_tumpy_argsort(gpu):
    from tallax_amd import tumpy as tnp
    a = np.random.default_rng(1).permutation(32).astype(np.int32).reshape(2, 16)
    assert np.array_equal(tnp.argsort(_dev(a), axis=-1).cpu().numpy(), np.argsort(a, axis=-1))


def test_tumpy_multidimensional_reshape(gpu):
    from tallax_amd import tumpy as tnp
    a = np.random.default_rng(2).integers(0, 100, (2, 2, 2, 16)).astype(np.int32)
    r = tnp.sort(_dev(a), axis=-1)
    assert tuple(r.shape) == (2, 2, 2, 16)
    assert np.array_equal(r.cpu().numpy(), np.sort(a, axis=-1))


def test_tumpy_1d_array(gpu):
    from tallax_amd import tumpy as tnp
    a = np.random.default_rng(3).integers(0, 100, (16,)).astype(np.int32)
    r = tnp.sort(_dev(a), axis=-1)
    assert tuple(r.shape) == (16,)
    assert np.array_equal(r.cpu().numpy(), np.sort(a))


def test_tumpy_descending(gpu):
    from tallax_amd import tumpy as tnp
    a = np.random.default_rng(4).integers(0, 100, (2, 16)).astype(np.int32)
    assert np.array_equal(tnp.sort(_dev(a), axis=-1, descending=True).cpu().numpy(), -np.sort(-a, axis=-1))
    args = tnp.argsort(_dev(a), axis=-1, descending=True).cpu().numpy()
    want = np.argsort(-a.astype(np.int64), axis=-1, kind="stable")   # stable=True: ties by ascending index
    assert np.array_equal(np.take_along_axis(a, args, -1), np.take_along_axis(a, want, -1))
    assert np.array_equal(args, want)


def test_tumpy_axis_validation(gpu):
    from tallax_amd import tumpy as tnp
    a = _dev(np.zeros((4, 4), np.float32))
    tnp.sort(a, axis=-1)
    tnp.sort(a, axis=1)
    with pytest.raises(ValueError, match="only supports sorting along the last axis"):
        tnp.sort(a, axis=0)
    with pytest.raises(ValueError):
        tnp.argsort(a, axis=0)


def test_tumpy_kind_and_order_ignored(gpu):
    from tallax_amd import tumpy as tnp
    a = _dev(np.array([3, 1, 2], np.int32))
    tnp.sort(a, kind="mergesort")
    tnp.argsort(a, kind="heapsort")
    tnp.sort(a, order="descending")
    tnp.argsort(a, order="something")


def test_tumpy_axis_none_flatten(gpu):
    from tallax_amd import tumpy as tnp
    a = np.random.default_rng(6).integers(0, 100, (2, 16)).astype(np.int32)
    r = tnp.sort(_dev(a), axis=None)
    assert tuple(r.shape) == (32,)
    assert np.array_equal(r.cpu().numpy(), np.sort(a, axis=None))
    args = tnp.argsort(_dev(a), axis=None)
    assert tuple(args.shape) == (32,)
    assert np.array_equal(args.cpu().numpy(), np.argsort(a.ravel(), kind="stable"))


# --------------------------------------------------------------------------- bitonic_topk_test.py
def _topk_input(shape, dtype, seed):
    rng = np.random.default_rng(seed)
    if dtype == "f32":
        return rng.standard_normal(shape).astype(np.float32)
    return rng.integers(0, 1000, shape).astype(np.int32)


@pytest.mark.parametrize("dtype", ["f32", "i32"])
@pytest.mark.parametrize("shape", [(8, 128), (16, 256), (13, 167), (256, 256), (173, 195)])
def test_bitonic_topk_axis1(gpu, shape, dtype):
    """tests/bitonic_topk_test.py:12-38: top-k with k = min(128, cols) along
    the last axis, float32 N(0, 1) and int32 randint(0, 1000) (many ties),
    through tax.top_k; bit-exact against the oracle (ties to the lowest
    index)."""
    from tallax_amd import tax
    _log(f"bitonic_topk_test {shape} {dtype}")
    x = _topk_input(shape, dtype, 0)
    k = min(128, shape[1])
    gv, gi = tax.top_k(torch.from_numpy(x).to(gpu), k)
    torch.cuda.synchronize()
    wv, wi = O.top_k(x, k, dtype)
    assert gv.dtype == (torch.int32 if dtype == "i32" else torch.float32)
    assert np.array_equal(gi.cpu().numpy(), wi)
    assert _same(gv.cpu().numpy(), wv)


@pytest.mark.parametrize("axis", [0, 1])
@pytest.mark.parametrize("dtype", ["f32", "i32"])
@pytest.mark.parametrize("shape", [(8, 128), (16, 256), (128, 8), (256, 16), (256, 256), (173, 195)])
def test_top1(gpu, shape, dtype, axis):
    """tests/bitonic_topk_test.py:41-102 (max_arrays along axis 0 or 1):
    the top-1 of every row (axis 1) or column (axis 0) through tax.top_k on
    the operand or its transpose, bit-exact against the oracle."""
    from tallax_amd import tax
    _log(f"top1 {shape} {dtype} axis={axis}")
    x = _topk_input(shape, dtype, 1 + axis)
    xt = x if axis == 1 else np.ascontiguousarray(x.T)
    gv, gi = tax.top_k(torch.from_numpy(xt).to(gpu), 1)
    torch.cuda.synchronize()
    wv, wi = O.top_k(xt, 1, dtype)
    assert np.array_equal(gi.cpu().numpy(), wi)
    assert _same(gv.cpu().numpy(), wv)
    assert np.array_equal(wv[:, 0], xt.max(axis=1))


def test_int32_topk_extremes_and_replace(gpu):
    """int32 rows holding iinfo.min / iinfo.max, rows that are all iinfo.min
    (their slots take the dtype's min, indices in order), a 151936-wide row
    (the wide sort route), and tallax_topk_replace's int32 replacement
    (converted toward zero, saturated)."""
    from tallax_amd import _lib, tax
    rng = np.random.default_rng(5)
    imin, imax = np.iinfo(np.int32).min, np.iinfo(np.int32).max
    x = rng.integers(-3, 4, (9, 300)).astype(np.int32)
    x[0, ::4] = imin
    x[1, ::5] = imax
    x[2] = imin
    x[3, :10] = rng.integers(0, 5, 10)
    x[3, 10:] = imin
    x[4] = rng.integers(imin, imax, 300, dtype=np.int64).astype(np.int32)
    for k in (1, 37, 128):
        gv, gi = tax.top_k(torch.from_numpy(x).to(gpu), k)
        wv, wi = O.top_k(x, k, "i32")
        assert np.array_equal(gi.cpu().numpy(), wi) and np.array_equal(gv.cpu().numpy(), wv)
    w = rng.integers(-50000, 50000, (4, 151936)).astype(np.int32)
    gv, gi = tax.top_k(torch.from_numpy(w).to(gpu), 50)
    wv, wi = O.top_k(w, 50, "i32")
    assert np.array_equal(gi.cpu().numpy(), wi) and np.array_equal(gv.cpu().numpy(), wv)
    rows, cols, k = x.shape[0], x.shape[1], 64
    kr = rng.integers(0, k + 1, rows).astype(np.int32)
    xd, krd = torch.from_numpy(x).to(gpu), torch.from_numpy(kr).to(gpu)
    for rv, want_rv in ((-1e12, imin), (7.9, 7), (-7.9, -7), (3e9, imax)):
        vals = torch.empty((rows, k), dtype=torch.int32, device=gpu)
        idx = torch.empty((rows, k), dtype=torch.int32, device=gpu)
        need = _lib.LIB.tallax_topk_workspace_size(rows, cols, k, _lib.I32)
        ws = torch.empty(need, dtype=torch.uint8, device=gpu)
        _lib.check(_lib.LIB.tallax_topk_replace(xd.data_ptr(), _lib.I32, rows, cols, k, krd.data_ptr(), rv,
                                                vals.data_ptr(), idx.data_ptr(), ws.data_ptr(), need,
                                                _lib.stream_of(xd)), "topk_replace")
        wv, wi = O.top_k(x, k, "i32")
        wv = np.where(np.arange(k)[None, :] < kr[:, None], wv, np.int32(want_rv))
        assert np.array_equal(idx.cpu().numpy(), wi) and np.array_equal(vals.cpu().numpy(), wv)
