"""GPU parity: tax.sort / tumpy.sort / tumpy.argsort through the C ABI against
the oracle's restatement of sort.py on identical seeded inputs (bit-exact
keys, indices and payloads), including config 2 (bf16 keys [256, 4096]
rounded to 1/16, stable argsort, then take_along_axis of an f32 array)."""
import numpy as np
import pytest
import torch

from oracle import tallax_oracle as O
from tests.gpu_util import bits, from_dev_vals, to_dev

pytestmark = pytest.mark.gpu


def _log(msg):
    print(msg, flush=True)


def _host(t: torch.Tensor) -> np.ndarray:
    if t.dtype == torch.bfloat16:
        return from_dev_vals(t)
    return t.cpu().numpy()


def _same(a: np.ndarray, b: np.ndarray) -> bool:
    if a.dtype == np.int32 or b.dtype == np.int32:
        return np.array_equal(a, b)
    return np.array_equal(bits(a), bits(b))


def _special_row(rng, cols):
    x = rng.standard_normal(cols).astype(np.float32)
    for v in (np.nan, -0.0, 0.0, np.inf, -np.inf, -np.nan):
        x[rng.integers(0, cols, max(1, cols // 50))] = v
    return x


def test_lds_atomics_return_in_lane_order(gpu):
    """The bf16 radix sort's stable ranks come from per-wave LDS counters: one
    atomic add per lane, whose returns must follow ascending lane order."""
    from tallax_amd import _lib
    nblocks = 512
    for ndig in (1, 3, 16, 256):
        _log(f"lds atomic order, {ndig} digits")
        d = torch.randint(0, 1 << 30, (nblocks * 256,), dtype=torch.int32, device=gpu)
        out = torch.empty_like(d)
        _lib.check(_lib.LIB.tallax_testing_lds_atomic_order(d.data_ptr(), nblocks, ndig, out.data_ptr(),
                                                            _lib.stream_of(d)), "lds_atomic_order")
        dig = (d.cpu().numpy().astype(np.int64) % ndig).reshape(-1, 64)
        want = np.zeros_like(dig)
        for lane in range(64):
            want[:, lane] = (dig[:, :lane] == dig[:, lane:lane + 1]).sum(axis=1)
        assert np.array_equal(out.cpu().numpy().reshape(-1, 64), want)


def test_config2_argsort_then_gather(gpu):
    from tallax_amd import tumpy
    _log("config 2: bf16 [256,4096] stable argsort + take_along_axis")
    rng = np.random.default_rng(1)
    keys = np.round(rng.standard_normal((256, 4096)) * 16) / 16
    keys = keys.astype(np.float32)
    vals = np.random.default_rng(2).standard_normal((256, 4096)).astype(np.float32)
    kd = to_dev(keys, "bf16", gpu)
    idx = tumpy.argsort(kd)
    got = tumpy.take_along_axis(torch.from_numpy(vals).to(gpu), idx, 1)
    torch.cuda.synchronize()
    (sk, want_idx), path = O.sort([O.round_to_dtype(keys, "bf16")], 1, is_stable=True, return_argsort=True,
                                  dtypes=["bf16"])
    assert path == "packed"
    assert np.array_equal(idx.cpu().numpy(), want_idx)
    assert np.array_equal(bits(got.cpu().numpy()), bits(O.take_along_axis(vals, want_idx, 1)))
    sorted_keys = tumpy.sort(kd)
    assert sorted_keys.dtype == torch.bfloat16
    assert _same(from_dev_vals(sorted_keys), sk)


@pytest.mark.parametrize("cols", [1, 7, 16, 17, 32, 255, 256, 1000, 4096, 5000, 16384])
@pytest.mark.parametrize("dtype", ["f32", "bf16", "i32"])
@pytest.mark.parametrize("descending", [False, True])
@pytest.mark.parametrize("stable,argsort", [(True, True), (False, True), (True, False), (False, False)])
def test_sort_one_key(gpu, cols, dtype, descending, stable, argsort):
    from tallax_amd import tax
    _log(f"sort {dtype} cols={cols} desc={descending} stable={stable} argsort={argsort}")
    rng = np.random.default_rng(cols * 3 + descending)
    rows = 5
    if dtype == "i32":
        x = rng.integers(-5, 5, (rows, cols)).astype(np.int32)
        x[0] = rng.integers(-2**31, 2**31, cols, dtype=np.int64).astype(np.int32)
        xd = torch.from_numpy(x).to(gpu)
        host = x
    else:
        x = np.round(rng.standard_normal((rows, cols)) * 8).astype(np.float32) / 8
        x[1] = _special_row(rng, cols)
        xd = to_dev(x, dtype, gpu)
        host = O.round_to_dtype(x, dtype)
    got = tax.sort(xd, num_keys=1, is_stable=stable, return_argsort=argsort, descending=descending)
    torch.cuda.synchronize()
    want, path = O.sort([host], 1, is_stable=stable, return_argsort=argsort, descending=descending,
                        dtypes=[dtype])
    assert len(got) == len(want)
    if dtype == "bf16":
        assert got[0].dtype == (torch.bfloat16 if path == "packed" else torch.float32)
    for g, w in zip(got, want):
        assert _same(_host(g), w)


@pytest.mark.parametrize("shape,dtype,descending,stable", [((70001, 8), "f32", True, True),
                                                           ((4099, 32), "bf16", True, False),
                                                           ((1000, 13), "i32", False, True)])
def test_sort_narrow_many_rows(gpu, shape, dtype, descending, stable):
    """Rows of at most 32 elements, one thread per row, across many workgroups."""
    from tallax_amd import tax
    _log(f"narrow sort {shape} {dtype} desc={descending} stable={stable}")
    rng = np.random.default_rng(shape[0])
    if dtype == "i32":
        x = rng.integers(-3, 3, shape).astype(np.int32)
        xd, host = torch.from_numpy(x).to(gpu), x
    else:
        x = np.round(rng.standard_normal(shape) * 4).astype(np.float32) / 4
        x[::97, ::3] = np.nan
        xd, host = to_dev(x, dtype, gpu), O.round_to_dtype(x, dtype)
    got = tax.sort(xd, num_keys=1, is_stable=stable, return_argsort=True, descending=descending)
    torch.cuda.synchronize()
    want, _ = O.sort([host], 1, is_stable=stable, return_argsort=True, descending=descending, dtypes=[dtype])
    for g, w in zip(got, want):
        assert _same(_host(g), w)


@pytest.mark.parametrize("cols", [3000, 24])   # 24: one thread per row, with a permutation in
@pytest.mark.parametrize("descending", [False, True])
def test_sort_two_keys_with_payloads(gpu, descending, cols):
    from tallax_amd import tax
    rng = np.random.default_rng(9)
    rows = 6
    k0 = rng.integers(0, 4, (rows, cols)).astype(np.int32)
    k1 = np.round(rng.standard_normal((rows, cols)) * 2).astype(np.float32) / 2
    k1[0, ::13] = np.nan
    pay_f = rng.standard_normal((rows, cols)).astype(np.float32)
    pay_b = rng.standard_normal((rows, cols)).astype(np.float32)
    ops = [torch.from_numpy(k0).to(gpu), torch.from_numpy(k1).to(gpu), torch.from_numpy(pay_f).to(gpu),
           to_dev(pay_b, "bf16", gpu)]
    got = tax.sort(ops, num_keys=2, return_argsort=True, descending=descending)
    torch.cuda.synchronize()
    want, _ = O.sort([k0, k1, pay_f, O.round_to_dtype(pay_b, "bf16")], 2, return_argsort=True,
                     descending=descending, dtypes=["i32", "f32", "f32", "bf16"])
    assert got[3].dtype == torch.bfloat16
    for g, w in zip(got, want):
        assert _same(_host(g), w)


def test_tumpy_axes_and_errors(gpu):
    from tallax_amd import tumpy
    rng = np.random.default_rng(3)
    x = rng.standard_normal((2, 3, 40)).astype(np.float32)
    xd = torch.from_numpy(x).to(gpu)
    s = tumpy.sort(xd)
    assert tuple(s.shape) == (2, 3, 40)
    assert np.array_equal(s.cpu().numpy(), np.sort(x, axis=-1))
    a = tumpy.argsort(xd, axis=None)
    assert tuple(a.shape) == (240,)
    assert np.array_equal(a.cpu().numpy(), np.argsort(x.reshape(-1), kind="stable"))
    d = tumpy.argsort(xd, descending=True)
    assert np.array_equal(d.cpu().numpy(), np.argsort(-x, axis=-1, kind="stable"))
    with pytest.raises(ValueError):
        tumpy.sort(xd, axis=0)
    from tallax_amd import tax
    with pytest.raises(ValueError):
        tax.sort([xd[0], xd[1, :2]], num_keys=1)
    with pytest.raises(ValueError):
        tax.sort(xd, num_keys=1)   # 3D


# Rows longer than 16384 (the reference's HBM substage route, sort.py:574-758):
# chunk sorts + merge passes through the workspace.  1, 2, 3 and 5 merge
# passes; ragged last chunks; the packed bf16 route up to 65536.
WIDE_COLS = [16385, 32768, 50001, 65536, 65537, 262147]
WIDE_MODES = [(False, True, True), (True, True, True), (True, False, True), (False, False, False)]


@pytest.mark.parametrize("cols", WIDE_COLS)
@pytest.mark.parametrize("dtype", ["f32", "bf16", "i32"])
@pytest.mark.parametrize("descending,stable,argsort", WIDE_MODES)
def test_sort_wide_rows(gpu, cols, dtype, descending, stable, argsort):
    from tallax_amd import tax
    _log(f"wide sort {dtype} cols={cols} desc={descending} stable={stable} argsort={argsort}")
    rng = np.random.default_rng(cols + 7 * descending + 3 * stable)
    rows = 3
    if dtype == "i32":
        x = rng.integers(-50, 50, (rows, cols)).astype(np.int32)
        x[0] = rng.integers(-2**31, 2**31, cols, dtype=np.int64).astype(np.int32)
        xd = torch.from_numpy(x).to(gpu)
        host = x
    else:
        x = np.round(rng.standard_normal((rows, cols)) * 8).astype(np.float32) / 8
        x[1] = _special_row(rng, cols)
        x[2, : cols // 2] = 0.5  # a long run of ties across chunk boundaries
        xd = to_dev(x, dtype, gpu)
        host = O.round_to_dtype(x, dtype)
    got = tax.sort(xd, num_keys=1, is_stable=stable, return_argsort=argsort, descending=descending)
    torch.cuda.synchronize()
    want, path = O.sort([host], 1, is_stable=stable, return_argsort=argsort, descending=descending,
                        dtypes=[dtype])
    assert len(got) == len(want)
    if dtype == "bf16":
        assert got[0].dtype == (torch.bfloat16 if path == "packed" else torch.float32)
    for g, w in zip(got, want):
        assert _same(_host(g), w)


# Rows of 25 to 56 chunks take the splitter merge with 16384-record buckets,
# longer ones the pairwise merge passes.
@pytest.mark.parametrize("cols", [500001, 1000003])
@pytest.mark.parametrize("descending,stable", [(True, True), (False, False)])
def test_sort_wide_long_rows(gpu, cols, descending, stable):
    from tallax_amd import tax
    _log(f"wide sort f32 cols={cols} desc={descending} stable={stable}")
    rng = np.random.default_rng(cols + descending)
    x = np.round(rng.standard_normal((2, cols)) * 8).astype(np.float32) / 8
    x[1, cols // 3: 2 * cols // 3] = -1.5  # ties across many chunks
    got = tax.sort(torch.from_numpy(x).to(gpu), num_keys=1, is_stable=stable, return_argsort=True,
                   descending=descending)
    torch.cuda.synchronize()
    want, _ = O.sort([x], 1, is_stable=stable, return_argsort=True, descending=descending)
    for g, w in zip(got, want):
        assert _same(_host(g), w)


def test_sort_wide_constant_and_nan_rows(gpu):
    from tallax_amd import tax
    cols = 40000
    x = np.zeros((3, cols), np.float32)
    x[0] = 1.25
    x[1] = np.nan
    x[2, ::2] = -0.0
    xd = torch.from_numpy(x).to(gpu)
    for desc in (False, True):
        got = tax.sort(xd, num_keys=1, is_stable=True, return_argsort=True, descending=desc)
        torch.cuda.synchronize()
        want, _ = O.sort([x], 1, is_stable=True, return_argsort=True, descending=desc)
        for g, w in zip(got, want):
            assert _same(_host(g), w)
        assert np.array_equal(got[1][0].cpu().numpy(), np.arange(cols, dtype=np.int32))


def test_sort_wide_prefill_shape_descending(gpu):
    """The reference's route for config 5's sort: softmax probabilities of a
    201088-wide row, descending argsort (sort.py:843 pads at the front)."""
    from tallax_amd import tax
    rng = np.random.default_rng(6)
    z = (rng.standard_normal((2, 201088)) * 2).astype(np.float32)
    p = np.exp(z - z.max(axis=1, keepdims=True))
    p = (p / p.sum(axis=1, keepdims=True)).astype(np.float32)
    got = tax.sort(torch.from_numpy(p).to(gpu), num_keys=1, is_stable=True, return_argsort=True, descending=True)
    torch.cuda.synchronize()
    want, _ = O.sort([p], 1, is_stable=True, return_argsort=True, descending=True)
    for g, w in zip(got, want):
        assert _same(_host(g), w)


@pytest.mark.parametrize("descending", [False, True])
def test_sort_wide_two_keys_with_payloads(gpu, descending):
    from tallax_amd import tax
    rng = np.random.default_rng(19)
    rows, cols = 2, 70000
    k0 = rng.integers(0, 4, (rows, cols)).astype(np.int32)
    k1 = np.round(rng.standard_normal((rows, cols)) * 2).astype(np.float32) / 2
    k1[0, ::13] = np.nan
    pay_f = rng.standard_normal((rows, cols)).astype(np.float32)
    pay_b = rng.standard_normal((rows, cols)).astype(np.float32)
    ops = [torch.from_numpy(k0).to(gpu), torch.from_numpy(k1).to(gpu), torch.from_numpy(pay_f).to(gpu),
           to_dev(pay_b, "bf16", gpu)]
    got = tax.sort(ops, num_keys=2, return_argsort=True, descending=descending)
    torch.cuda.synchronize()
    want, _ = O.sort([k0, k1, pay_f, O.round_to_dtype(pay_b, "bf16")], 2, return_argsort=True,
                     descending=descending, dtypes=["i32", "f32", "f32", "bf16"])
    for g, w in zip(got, want):
        assert _same(_host(g), w)


def test_tumpy_flattened_wide(gpu):
    from tallax_amd import tumpy
    rng = np.random.default_rng(23)
    x = np.round(rng.standard_normal((4, 30000)) * 4).astype(np.float32) / 4
    xd = torch.from_numpy(x).to(gpu)
    a = tumpy.argsort(xd, axis=None)
    s = tumpy.sort(xd, axis=None)
    torch.cuda.synchronize()
    assert np.array_equal(a.cpu().numpy(), np.argsort(x.reshape(-1), kind="stable"))
    assert np.array_equal(s.cpu().numpy(), np.sort(x.reshape(-1)))


@pytest.mark.parametrize("cols", [3000, 40000])
@pytest.mark.parametrize("descending", [False, True])
def test_sort_many_keys(gpu, cols, descending):
    """Three and four keys (lexicographic, sort.py:768-929): LSD passes with
    the permutation carried along; the third and later keys come back
    standardised and decoded like the first two (NaN payload, -0 -> +0,
    bf16 keys as float32)."""
    from tallax_amd import tax
    rng = np.random.default_rng(cols + descending)
    rows = 3
    k0 = rng.integers(0, 3, (rows, cols)).astype(np.int32)
    k1 = np.round(rng.standard_normal((rows, cols))).astype(np.float32)
    k2 = np.round(rng.standard_normal((rows, cols)) * 2).astype(np.float32) / 2
    k2[0, ::7] = np.nan
    k2[1, ::5] = -0.0
    k3 = np.round(rng.standard_normal((rows, cols)) * 4).astype(np.float32) / 4
    pay = rng.standard_normal((rows, cols)).astype(np.float32)
    for nk, ops_h, dts in [(3, [k0, k1, k2, pay], ["i32", "f32", "f32", "f32"]),
                           (4, [k1, k0, k2, O.round_to_dtype(k3, "bf16"), pay], ["f32", "i32", "f32", "bf16", "f32"])]:
        ops = [torch.from_numpy(o).to(gpu) if d != "bf16" else to_dev(o, "bf16", gpu) for o, d in zip(ops_h, dts)]
        got = tax.sort(ops, num_keys=nk, is_stable=True, return_argsort=True, descending=descending)
        torch.cuda.synchronize()
        want, _ = O.sort(ops_h, nk, is_stable=True, return_argsort=True, descending=descending, dtypes=dts)
        assert len(got) == len(want)
        for g, w in zip(got, want):
            assert _same(_host(g), w)
