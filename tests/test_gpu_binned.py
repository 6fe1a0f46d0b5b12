"""GPU parity: tax.top_dynamic_k (binned, with and without
guarantee_convergence's bin-packing merge) through the C ABI against the
oracle on identical seeded inputs (bit-exact values, indices, valid, depths and
cutoffs), with config 3's recall@50 of the approximate result against the
exact one reported."""
import numpy as np
import pytest
import torch

from oracle import tallax_oracle as O
from tests.gpu_util import bits, from_dev_vals, to_dev

pytestmark = pytest.mark.gpu


def _log(msg):
    print(msg, flush=True)


@pytest.fixture(params=[0, 1], ids=["candidates", "scan"])
def binned_mode(request):
    """Runs a test once with the candidate path (rows settled from the exact
    kernel's per-segment top-128 where they suffice, the rest scanned) and
    once with the full scan for every row; both must match the oracle.  The
    path goes to the testing entry point tallax_testing_top_dynamic_k_path."""
    return request.param


def _dyn(x, k, max_k, path, block_token=8, num_bins=128, bins_topm_schedule=None, replace_val=None):
    from tallax_amd import tax
    return tax._top_dynamic_k(x, k, max_k, block_token, num_bins, 32, bins_topm_schedule, False, replace_val,
                              False, None, path)


def _check(got, want):
    gv, gi, gvalid, gd, gc = got
    wv, wi, wvalid, wd, wc = want
    assert bool(gvalid.item()) == wvalid
    assert np.array_equal(gd.cpu().numpy(), wd)
    assert np.array_equal(bits(gc.cpu().numpy()), bits(wc))
    assert np.array_equal(gi.cpu().numpy(), wi)
    assert np.array_equal(bits(from_dev_vals(gv)), bits(wv))


def test_config3_approx_and_recall(gpu, binned_mode):
    from tallax_amd import tax
    _log("config 3 approximate: f32 [128,151936] + spikes, k=50")
    rng = np.random.default_rng(3)
    x = (rng.standard_normal((128, 151936)) * 2).astype(np.float32)
    for r in range(128):
        x[r, rng.choice(151936, 32, replace=False)] = 8.0
    xd = torch.from_numpy(x).to(gpu)
    got = _dyn(xd, 50, 50, binned_mode)
    torch.cuda.synchronize()
    want = O.top_dynamic_k(x, 50, 50)
    _check(got, want)
    ev, ei = O.top_k(x, 50)
    gi = got[1].cpu().numpy()
    recall = np.mean([len(set(gi[r]) & set(ei[r])) / 50 for r in range(128)])
    _log(f"recall@50 of approximate vs exact: {recall:.4f}")
    assert recall == 1.0 and bool(got[2].item())


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("rows,cols,max_k,num_bins,block_token,schedule", [
    (16, 20000, 64, 128, 8, None),
    (8, 5000, 128, 256, 8, None),
    (12, 3000, 20, 64, 4, (3, 6)),
    (8, 300, 32, 128, 8, (2, 4, 9)),     # short rows: fillers at depth
    (16, 50000, 8, 512, 8, (2,)),        # one-step schedule
    (16, 151936, 50, 128, 8, None),      # config-3 rows with heavy ties: candidates and scan mixed
])
def test_top_dynamic_k_parity(gpu, binned_mode, dtype, rows, cols, max_k, num_bins, block_token, schedule):
    from tallax_amd import tax
    _log(f"top_dynamic_k {dtype} [{rows},{cols}] max_k={max_k} bins={num_bins} bt={block_token} sched={schedule}")
    rng = np.random.default_rng(rows * cols + max_k)
    x = np.round(rng.standard_normal((rows, cols)) * 16).astype(np.float32) / 16   # many ties
    x[0, ::5] = np.nan
    x[1, ::3] = -np.inf
    x[2, 1::4] = O.dtype_min(dtype)
    k = rng.integers(1, max_k + 1, rows).astype(np.int32)
    xd = to_dev(x, dtype, gpu)
    got = _dyn(xd, torch.from_numpy(k).to(gpu), max_k, binned_mode, block_token=block_token, num_bins=num_bins,
               bins_topm_schedule=schedule, replace_val=-1e12)
    torch.cuda.synchronize()
    want = O.top_dynamic_k(O.round_to_dtype(x, dtype), k, max_k, block_token=block_token, num_bins=num_bins,
                           schedule=schedule, replace_val=-1e12, dtype=dtype)
    _check(got, want)


_ORACLE_CACHE = {}


def _unconverged_rows(rows, cols, num_bins, spike_rows, nspikes, seed):
    """Untied Gaussian rows; rows in spike_rows get nspikes large distinct
    values all in bin 0 (columns = 0 mod num_bins), so the per-bin top-(m-1)
    lists cannot hold k of them at any shallow step: those rows (and their
    blocks) never converge."""
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal((rows, cols)) * 2).astype(np.float32)
    nspikes = min(nspikes, cols // num_bins)
    for r in spike_rows:
        x[r, rng.choice(cols // num_bins, nspikes, replace=False) * num_bins] = 50.0 + rng.random(nspikes)
    return x


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("replace", [None, -1e12], ids=["no_replace", "replace"])
@pytest.mark.parametrize("rows,cols,max_k,num_bins,block_token,schedule,spike_rows", [
    (16, 3000, 32, 64, 8, (3, 6, 12), (5, 6)),           # depth_upper 16 > m_final 12
    (16, 3000, 32, 64, 4, (2, 3, 6, 12), (9,)),           # blocks stop at different steps
    (64, 151936, 50, 128, 8, (2, 5, 9), (3, 17, 40)),     # config-3 width, some blocks unconverged
])
def test_top_dynamic_k_unconverged_blocks(gpu, binned_mode, dtype, replace, rows, cols, max_k, num_bins,
                                          block_token, schedule, spike_rows):
    """Blocks that never converge (depth max_k, valid False) next to blocks
    that stop early: the ranks a block never evaluated stay finfo.min
    (top_k.py:241-243, 250-315, 333-364), bit-exact against the oracle, which
    is pinned by the literal block-by-block restatement in test_oracle.py."""
    _log(f"top_dynamic_k unconverged {dtype} [{rows},{cols}] max_k={max_k} bins={num_bins} bt={block_token} "
         f"sched={schedule} replace={replace} path={binned_mode}")
    x = O.round_to_dtype(_unconverged_rows(rows, cols, num_bins, spike_rows, 2 * max_k, rows + cols), dtype)
    rng = np.random.default_rng(cols)
    k = rng.integers(max_k // 2, max_k + 1, rows).astype(np.int32)
    for r in spike_rows:
        k[r] = max_k
    xd = to_dev(x, dtype, gpu)
    got = _dyn(xd, torch.from_numpy(k).to(gpu), max_k, binned_mode, block_token=block_token, num_bins=num_bins,
               bins_topm_schedule=schedule, replace_val=replace)
    torch.cuda.synchronize()
    key = (dtype, replace, rows, cols, max_k, num_bins, block_token, schedule, spike_rows)
    if key not in _ORACLE_CACHE:   # the same inputs run on both paths
        _ORACLE_CACHE[key] = O.top_dynamic_k(x, k, max_k, block_token=block_token, num_bins=num_bins,
                                             schedule=schedule, replace_val=replace, dtype=dtype)
    want = _ORACLE_CACHE[key]
    assert not want[2] and (want[3][list(spike_rows)] == max_k).all()
    _check(got, want)


@pytest.mark.parametrize("rows,block_token", [(2048, 8), (2048, 2048), (1536, 512)])
def test_top_dynamic_k_many_rows_and_wide_blocks(gpu, binned_mode, rows, block_token):
    """More rows than one finish workgroup has threads (the separate finish
    kernel) and blocks wider than it: per-block last steps over any
    block_token."""
    _log(f"top_dynamic_k rows={rows} block_token={block_token} path={binned_mode}")
    cols, max_k, nb, sched = 1000, 16, 32, (2, 4, 7)
    x = _unconverged_rows(rows, cols, nb, (7, rows - 1), 24, rows + block_token)
    rng = np.random.default_rng(block_token)
    k = rng.integers(1, max_k + 1, rows).astype(np.int32)
    got = _dyn(torch.from_numpy(x).to(gpu), torch.from_numpy(k).to(gpu), max_k, binned_mode,
               block_token=block_token, num_bins=nb, bins_topm_schedule=sched, replace_val=None)
    torch.cuda.synchronize()
    want = O.top_dynamic_k(x, k, max_k, block_token=block_token, num_bins=nb, schedule=sched)
    _check(got, want)


def _merge_rows(rows, cols, num_bins, spike_rows, spike_bins, nspikes, seed, masked_rows=()):
    """Untied Gaussian rows; rows in spike_rows get nspikes large distinct
    values spread over the bins spike_bins, so that their blocks cannot
    converge at a shallow depth and go through the bin-packing merge; rows in
    masked_rows are -inf but for a few values, with three spikes in bin 3."""
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal((rows, cols)) * 2).astype(np.float32)
    per = cols // num_bins
    for r in spike_rows:
        for j, b in enumerate(spike_bins):
            n = min(nspikes // len(spike_bins), per)
            x[r, rng.choice(per, n, replace=False) * num_bins + b] = 40.0 + 10 * j + rng.random(n)
    for r in masked_rows:
        x[r] = -np.inf
        x[r, rng.choice(cols, 12, replace=False)] = rng.standard_normal(12)
        x[r, [3, 3 + num_bins, 3 + 2 * num_bins]] = [9.0, 8.0, 7.0]
    return x


@pytest.mark.parametrize("replace", [None, -1e12], ids=["no_replace", "replace"])
@pytest.mark.parametrize("dtype,rows,cols,max_k,num_bins,block_token,schedule,spikes,masked", [
    ("f32", 16, 3000, 32, 128, 8, (3, 6), ((5, 6), (0, 9), 32), ()),          # P = 8
    ("bf16", 64, 50000, 128, 256, 8, (5, 9), ((3, 17, 40), (0, 1, 2, 3), 300), (41,)),  # the sampler's call, P = 16
    ("bf16", 8, 700, 16, 256, 4, (2,), ((), (), 0), tuple(range(8))),          # packed slots past the row's end
    ("f32", 32, 128256, 128, 128, 8, (2,), ((1, 9), (5,), 200), ()),           # P = num_bins: whole rows packed
])
def test_top_dynamic_k_merge_parity(gpu, binned_mode, replace, dtype, rows, cols, max_k, num_bins, block_token,
                                    schedule, spikes, masked):
    """guarantee_convergence=True with a last depth below max_k: blocks that
    did not converge go through the bin-packing merge
    (_merge_unconverged_bins_top_k, top_k.py:108-200), bit-exact against the
    oracle, which is pinned by the tile-level literal restatement in
    test_oracle.py.  With P == num_bins the merged rows are the exact top-k."""
    from tallax_amd import tax
    _log(f"top_dynamic_k merge {dtype} [{rows},{cols}] max_k={max_k} bins={num_bins} bt={block_token} "
         f"sched={schedule} replace={replace} path={binned_mode}")
    x = O.round_to_dtype(_merge_rows(rows, cols, num_bins, *spikes, rows + cols, masked), dtype)
    rng = np.random.default_rng(cols + 1)
    k = rng.integers(max_k // 2, max_k + 1, rows).astype(np.int32)
    for r in spikes[0]:
        k[r] = max_k
    xd = to_dev(x, dtype, gpu)
    gv, gi = tax._top_dynamic_k(xd, torch.from_numpy(k).to(gpu), max_k, block_token, num_bins, 32, schedule, True,
                                replace, False, None, binned_mode)
    torch.cuda.synchronize()
    key = ("merge", dtype, replace, rows, cols, max_k, num_bins, block_token, schedule)
    if key not in _ORACLE_CACHE:   # the same inputs run on both paths
        conv = O.top_dynamic_k(x, k, max_k, block_token=block_token, num_bins=num_bins, schedule=schedule,
                               dtype=dtype)
        _ORACLE_CACHE[key] = (O.top_dynamic_k(x, k, max_k, block_token=block_token, num_bins=num_bins,
                                              schedule=schedule, replace_val=replace, dtype=dtype,
                                              guarantee_convergence=True), conv)
    (wv, wi), conv = _ORACLE_CACHE[key]
    unconv = np.repeat((conv[3].reshape(-1, block_token) == max_k).any(axis=1), block_token)
    _log(f"rows in unconverged blocks: {int(unconv.sum())} of {rows}")
    assert unconv.any()
    assert np.array_equal(gi.cpu().numpy(), wi)
    assert np.array_equal(bits(from_dev_vals(gv)), bits(wv))
    if O.packed_bins(max_k, schedule[-1]) == num_bins and replace is None:
        ev, ei = O.top_k(x, max_k, dtype)
        assert np.array_equal(wi[unconv], ei[unconv])


def test_top_dynamic_k_sampler_call_on_config4_is_exact(gpu):
    """The reference sampler's top-k stage (sampling.py:283-290:
    top_dynamic_k(max_k=128, guarantee_convergence=True, num_bins=256,
    bins_topm_schedule=(5, 9), replace_val)) on config 4's logits: every
    block converges, so the result is the exact top-k inside k[row], which is
    what the fused sampler computes."""
    from tallax_amd import tax
    rng = np.random.default_rng(4)
    x = (rng.standard_normal((256, 128256)) * 3).astype(np.float32)
    k = rng.integers(1, 1025, 256).clip(max=128).astype(np.int32)
    xd = to_dev(x, "bf16", gpu)
    vals, idx = tax.top_dynamic_k(xd, torch.from_numpy(k).to(gpu), 128, num_bins=256, bins_topm_schedule=(5, 9),
                                  guarantee_convergence=True, replace_val=-1e12)
    torch.cuda.synchronize()
    hv = O.round_to_dtype(x, "bf16")
    wv, wi = O.top_dynamic_k(hv, k, 128, num_bins=256, schedule=(5, 9), replace_val=-1e12, dtype="bf16",
                             guarantee_convergence=True)
    assert np.array_equal(idx.cpu().numpy(), wi)
    assert np.array_equal(bits(from_dev_vals(vals)), bits(wv))
    ev, ei = O.top_k(hv, 128, dtype="bf16")
    inside = np.arange(128)[None, :] < k[:, None]
    assert np.array_equal(np.where(inside, wi, -2), np.where(inside, ei, -2))


def test_top_dynamic_k_sampler_call_unclipped_k_on_config4(gpu):
    """The reference sampler's own top-k call (sampling.py:283-290, 333-336)
    with the per-row k it really passes: tpu_sampling_metadata.top_k is not
    clipped, so k[row] in [1, 1024] enters the convergence test
    (top_k.py:298) and most blocks cannot converge, reaching the bin-packing
    merge (top_k.py:317-331).  Bit-exact against the oracle on the same call;
    the merged result equals the exact top-128 inside min(k, 128); and the
    reference route (this top-k, then top_p_and_sample) gives the fused
    sampler's tokens."""
    from tallax_amd import sampling, tax
    _log("config 4 sampler top-k call, unclipped k in [1, 1024]")
    rng = np.random.default_rng(4)
    x = (rng.standard_normal((256, 128256)) * 3).astype(np.float32)
    k = rng.integers(1, 1025, 256).astype(np.int32)
    temp = rng.uniform(0.5, 1.5, 256).astype(np.float32)
    topp = rng.uniform(0.7, 1.0, 256).astype(np.float32)
    xd = to_dev(x, "bf16", gpu)
    vals, idx = tax.top_dynamic_k(xd, torch.from_numpy(k).to(gpu), 128, num_bins=256, bins_topm_schedule=(5, 9),
                                  guarantee_convergence=True, replace_val=-1e12)
    torch.cuda.synchronize()
    hv = O.round_to_dtype(x, "bf16")
    wv, wi = O.top_dynamic_k(hv, k, 128, num_bins=256, schedule=(5, 9), replace_val=-1e12, dtype="bf16",
                             guarantee_convergence=True)
    assert np.array_equal(idx.cpu().numpy(), wi)
    assert np.array_equal(bits(from_dev_vals(vals)), bits(wv))
    _, _, valid, depths, _ = O.top_dynamic_k(hv, k, 128, num_bins=256, schedule=(5, 9), dtype="bf16")
    unconv = (depths.reshape(-1, 8) == 128).any(axis=1)
    _log(f"blocks through the merge: {int(unconv.sum())} of 32; rows at depth 128: {int((depths == 128).sum())}")
    assert not valid and unconv.any()
    ev, ei = O.top_k(hv, 128, dtype="bf16")
    inside = np.arange(128)[None, :] < np.minimum(k, 128)[:, None]
    assert np.array_equal(np.where(inside, wi, -2), np.where(inside, ei, -2))
    key = (0, 1234)
    route = O.top_p_and_sample(wv, wi, key, topp, temp, 128256, -1e12)
    meta = sampling.SamplingMetadata(torch.from_numpy(k), torch.from_numpy(topp), torch.from_numpy(temp))
    tok = sampling.sample(key, xd, meta)
    torch.cuda.synchronize()
    assert np.array_equal(tok.cpu().numpy(), route)


def _int32_cases():
    imin = np.iinfo(np.int32).min
    rng = np.random.default_rng(31)
    a = rng.integers(0, 1000, (16, 20000)).astype(np.int32)           # heavy ties
    a[3, ::7] = imin
    yield "ties", a, rng.integers(1, 65, 16).astype(np.int32), 64, 128, 8, None, False
    b = rng.integers(-2 ** 31 + 1, 2 ** 31 - 1, (16, 3000), dtype=np.int64).astype(np.int32)
    for r in (5, 6):                                                    # unconverged block 0
        b[r, rng.choice(3000 // 128, 20, replace=False) * 128] = 2 ** 31 - 1 - rng.permutation(20)
    yield "unconverged, merge", b, np.full(16, 32, np.int32), 32, 128, 8, (3, 6), True
    yield "unconverged, no merge", b, np.full(16, 32, np.int32), 32, 128, 8, (3, 6), False
    c = np.full((8, 700), imin, np.int32)
    for r in range(8):
        c[r, rng.choice(700, 6 + r, replace=False)] = rng.integers(-1000, 1000, 6 + r)
    yield "mostly iinfo.min", c, rng.integers(1, 17, 8).astype(np.int32), 16, 32, 4, (2, 5), False


@pytest.mark.parametrize("replace", [None, -1e12, 7.9], ids=["no_replace", "replace_min", "replace_7"])
@pytest.mark.parametrize("case", list(_int32_cases()), ids=lambda c: c[0] if isinstance(c, tuple) else str(c))
def test_top_dynamic_k_int32(gpu, binned_mode, case, replace):
    """int32 logits (the reference's dtype-generic path: iinfo.min bins,
    utils.py:48-56): values, indices, valid, depths and int32 cutoff_vals
    bit-exact against the oracle, which the literal block restatement pins
    for int32 in test_oracle.py.  int32 always takes the full scan."""
    from tallax_amd import tax
    name, x, k, max_k, nb, bt, sched, gc = case
    _log(f"top_dynamic_k int32 {name} [{x.shape[0]},{x.shape[1]}] replace={replace} path={binned_mode}")
    out = tax._top_dynamic_k(torch.from_numpy(x).to(gpu), torch.from_numpy(k).to(gpu), max_k, bt, nb, 32, sched,
                             gc, replace, False, None, binned_mode)
    torch.cuda.synchronize()
    want = O.top_dynamic_k(x, k, max_k, block_token=bt, num_bins=nb, schedule=sched, replace_val=replace,
                           dtype="i32", guarantee_convergence=gc)
    assert out[0].dtype == torch.int32
    assert np.array_equal(out[1].cpu().numpy(), want[1])
    assert np.array_equal(out[0].cpu().numpy(), want[0])
    if not gc:
        assert bool(out[2].item()) == want[2]
        assert np.array_equal(out[3].cpu().numpy(), want[3])
        assert out[4].dtype == torch.int32 and np.array_equal(out[4].cpu().numpy(), want[4])


def test_top_dynamic_k_errors(gpu):
    from tallax_amd import tax
    x = torch.zeros((12, 100), device=gpu)
    with pytest.raises(ValueError):
        tax.top_dynamic_k(x, 4, 4, block_token=8)
    with pytest.raises(NotImplementedError):
        tax.top_dynamic_k(x[:8], 4, 129)
    with pytest.raises(ValueError):
        tax.top_dynamic_k(x[:8], 4, 8, bins_topm_schedule=(1,), guarantee_convergence=True)
    with pytest.raises(NotImplementedError):
        tax.top_dynamic_k(x[:8], 4, 8, num_bins=64, bins_topm_schedule=(2,), guarantee_convergence=True)


def test_candidates_settle_config3_rows(gpu):
    """White-box: on config 3 the per-segment candidates settle every row (the
    covered flag follows the candidate lists at the front of the workspace)."""
    import ctypes
    from tallax_amd import _lib, schedule as sch
    rng = np.random.default_rng(3)
    rows, cols = 128, 151936
    x = (rng.standard_normal((rows, cols)) * 2).astype(np.float32)
    for r in range(rows):
        x[r, rng.choice(cols, 32, replace=False)] = 8.0
    xd = torch.from_numpy(x).to(gpu)
    steps = sch.topm_schedule(50, 128, 8, None)
    arr = (ctypes.c_int32 * len(steps))(*steps)
    need = _lib.LIB.tallax_top_dynamic_k_workspace_size(rows, 128, arr, len(steps))
    ws = torch.zeros(need, dtype=torch.uint8, device=gpu)
    k = torch.full((rows,), 50, dtype=torch.int32, device=gpu)
    vals = torch.empty((rows, 50), dtype=torch.float32, device=gpu)
    idx = torch.empty((rows, 50), dtype=torch.int32, device=gpu)
    valid = torch.empty(1, dtype=torch.int32, device=gpu)
    depths = torch.empty(rows, dtype=torch.int32, device=gpu)
    cutoff = torch.empty(rows, dtype=torch.float32, device=gpu)
    _lib.check(_lib.LIB.tallax_top_dynamic_k(
        xd.data_ptr(), _lib.F32, rows, cols, k.data_ptr(), 50, 8, 128, arr, len(steps), 0, 0, 0.0, vals.data_ptr(),
        idx.data_ptr(), valid.data_ptr(), depths.data_ptr(), cutoff.data_ptr(), ws.data_ptr(), need,
        _lib.stream_of(xd)), "top_dynamic_k")
    torch.cuda.synchronize()
    off = rows * 32 * 128 * 8
    covered = ws[off:off + rows * 4].view(torch.int32).cpu().numpy()
    _log(f"rows settled by candidates: {int(covered.sum())} of {rows}")
    assert covered.sum() == rows
    want = O.top_dynamic_k(x, 50, 50)
    assert np.array_equal(idx.cpu().numpy(), want[1])
    assert np.array_equal(depths.cpu().numpy(), want[3])
