"""GPU parity: take_along_axis and cumsum through the C ABI against the oracle
on identical seeded inputs (bit-exact), plus cumsum against float64 within
the 1e-5 relative tolerance BASELINE states for fp32 scans."""
import numpy as np
import pytest
import torch

from oracle import tallax_oracle as O
from tests.gpu_util import bits, from_dev_vals, to_dev

pytestmark = pytest.mark.gpu


def _log(msg):
    print(msg, flush=True)


# --------------------------------------------------------------------------- take_along_axis
@pytest.mark.parametrize("dtype", ["f32", "bf16", "i32"])
@pytest.mark.parametrize("shape_v,shape_i,axis", [
    ((256, 4096), (256, 4096), 1),      # config 2's gather (values staged in LDS)
    ((16, 40000), (16, 300), 1),        # long rows: direct global gather
    ((512, 20480), (512, 700), 1),      # f32 rows of exactly 80 KiB staged in LDS (>= 512 rows)
    ((8, 40960), (8, 40960), 1),        # rows beyond LDS: XCD-ordered chunks
    ((9, 70000), (9, 20000), 1),        # XCD-ordered chunks, 9 rows (two XCD rounds)
    ((3, 100003), (3, 16384), 1),       # XCD chunks at the smallest index row it takes
    ((7, 130), (7, 50), 1),             # ragged
    ((1000, 33), (200, 33), 0),         # axis 0
    ((5, 1), (5, 9), 1),
])
def test_take_along_axis_parity(gpu, dtype, shape_v, shape_i, axis):
    from tallax_amd import tumpy
    _log(f"take_along_axis {dtype} {shape_v} {shape_i} axis={axis}")
    rng = np.random.default_rng(sum(shape_v) + axis)
    ext = shape_v[axis]
    idx = rng.integers(-3, ext + 3, shape_i).astype(np.int32)
    idx.flat[::7] = -1            # negative and out-of-range indices on every row
    idx.flat[3::11] = ext
    idx.flat[5::13] = 2**31 - 1
    if dtype == "i32":
        v = rng.integers(-2**31, 2**31, shape_v, dtype=np.int64).astype(np.int32)
        vd = torch.from_numpy(v).to(gpu)
        want = O.take_along_axis(v, idx, axis)
    else:
        v = (rng.standard_normal(shape_v) * 3).astype(np.float32)
        vd = to_dev(v, dtype, gpu)
        want = O.take_along_axis(O.round_to_dtype(v, dtype), idx, axis)
    got = tumpy.take_along_axis(vd, torch.from_numpy(idx).to(gpu), axis)
    torch.cuda.synchronize()
    assert got.dtype == vd.dtype and tuple(got.shape) == shape_i
    g = got.cpu().numpy() if dtype == "i32" else from_dev_vals(got)
    if dtype == "i32":
        assert np.array_equal(g, want)
    else:
        assert np.array_equal(bits(g), bits(want))
    # out-of-range and negative indices give exactly +0
    bad = (idx < 0) | (idx >= ext)
    assert bad.any()
    zero_bits = g[bad] if dtype == "i32" else bits(g)[bad]
    assert np.all(zero_bits == 0)


def test_take_along_axis_errors(gpu):
    from tallax_amd import tumpy
    v = torch.zeros((4, 8), device=gpu)
    with pytest.raises(ValueError):
        tumpy.take_along_axis(v, torch.zeros((3, 2), dtype=torch.int32, device=gpu), 1)
    with pytest.raises(ValueError):
        tumpy.take_along_axis(v.reshape(-1), torch.zeros((4,), dtype=torch.int32, device=gpu), 0)


# --------------------------------------------------------------------------- cumsum
SHAPES = [(1024, 2048), (3, 200), (5, 130), (2, 20000), (9, 128), (1, 1), (300, 7), (17, 1000)]


@pytest.mark.parametrize("shape", SHAPES)
@pytest.mark.parametrize("axis", [0, 1])
@pytest.mark.parametrize("reverse", [False, True])
def test_cumsum_parity_f32(gpu, shape, axis, reverse):
    from tallax_amd import tax
    _log(f"cumsum f32 {shape} axis={axis} reverse={reverse}")
    rng = np.random.default_rng(shape[0] * 31 + shape[1] + axis)
    x = rng.standard_normal(shape).astype(np.float32)
    x.flat[::97] = -0.0
    got = tax.cumsum(torch.from_numpy(x).to(gpu), axis, reverse=reverse)
    torch.cuda.synchronize()
    g = got.cpu().numpy()
    want = O.cumsum(x, axis, reverse)
    assert np.array_equal(bits(g), bits(want))
    # against float64 (the truth), BASELINE's 1e-5 relative for fp32 scans
    a = np.flip(x, axis) if reverse else x
    r64 = np.cumsum(a.astype(np.float64), axis=axis)
    r64 = np.flip(r64, axis) if reverse else r64
    scale = np.maximum(np.abs(r64), np.cumsum(np.abs(a.astype(np.float64)), axis=axis).max())
    assert np.all(np.abs(g - r64) <= 1e-5 * scale)


# Each launch route of tallax_cumsum: one workgroup per row (>= 256 rows of
# >= 64 tiles; 65 and 71 tiles leave a partial chunk of 64), and the three
# launches (tile totals -> chain -> rescan) with one line per chain workgroup,
# several lines per workgroup (gl 2 and 4, the last group partial), and
# chains longer than one staged block of totals; and one thread per row for
# rows of at most 16 elements (17 to 65 take a wave per tile).
ROUTES = [((256, 9000), 1), ((300, 8320), 1), ((255, 9000), 1), ((256, 1500), 1), ((1101, 1900), 1),
          ((1, 2200000), 1), ((140000, 2), 0), ((66000, 513), 0), ((5, 7), 0), ((9, 1), 0),
          ((100000, 16), 1), ((70001, 5), 1), ((3, 17), 1), ((30000, 64), 1), ((20000, 50), 1),
          ((5, 65), 1)]


@pytest.mark.parametrize("shape,axis", ROUTES)
@pytest.mark.parametrize("reverse", [False, True])
def test_cumsum_parity_routes(gpu, shape, axis, reverse):
    from tallax_amd import tax
    _log(f"cumsum route {shape} axis={axis} reverse={reverse}")
    rng = np.random.default_rng(shape[0] * 7 + shape[1] + axis)
    x = rng.standard_normal(shape).astype(np.float32)
    x.flat[::89] = -0.0
    got = tax.cumsum(torch.from_numpy(x).to(gpu), axis, reverse=reverse).cpu().numpy()
    assert np.array_equal(bits(got), bits(O.cumsum(x, axis, reverse)))


def test_cumsum_rejects_overlap(gpu):
    from tallax_amd import _lib
    x = torch.zeros((4, 300), device=gpu)
    rc = _lib.LIB.tallax_cumsum(x.data_ptr(), _lib.F32, 4, 300, 1, 0, x.data_ptr() + 512,
                                _lib.stream_of(x))
    assert rc != 0 and b"overlap" in _lib.LIB.tallax_last_error()


@pytest.mark.parametrize("shape", [(64, 5000), (300, 9), (4, 128), (256, 9000), (40000, 3)])
@pytest.mark.parametrize("axis", [0, 1])
@pytest.mark.parametrize("reverse", [False, True])
def test_cumsum_int32_exact(gpu, shape, axis, reverse):
    from tallax_amd import tax
    rng = np.random.default_rng(7 + axis)
    x = rng.integers(-2**31, 2**31, shape, dtype=np.int64).astype(np.int32)   # wraps
    got = tax.cumsum(torch.from_numpy(x).to(gpu), axis, reverse=reverse).cpu().numpy()
    a = np.flip(x, axis) if reverse else x
    r = np.cumsum(a.astype(np.int64), axis=axis)
    r = np.flip(r, axis) if reverse else r
    assert np.array_equal(got, (r & 0xFFFFFFFF).astype(np.uint32).view(np.int32))


def test_cumsum_probability_rows(gpu):
    """Config 5's scan: sorted softmax probabilities [1024, 2048]."""
    from tallax_amd import tax
    rng = np.random.default_rng(6)
    p = rng.dirichlet(np.ones(4096), size=1024).astype(np.float32)
    p = -np.sort(-p, axis=1)[:, :2048].copy()
    got = tax.cumsum(torch.from_numpy(p).to(gpu), 1).cpu().numpy()
    assert np.array_equal(bits(got), bits(O.cumsum(p, 1)))
    np.testing.assert_allclose(got, np.cumsum(p.astype(np.float64), 1), rtol=1e-5, atol=0)
