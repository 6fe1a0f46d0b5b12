"""GPU: tallax_fused_topk_topp_sample_noalloc (static device scratch, no
allocation) through the C ABI against tallax_fused_topk_topp_sample with a
caller workspace: identical tokens on two calls in a row, the second with a
smaller input, for segmented plans (which use the scratch) and a whole-row
plan (which does not)."""
import numpy as np
import pytest
import torch

from tests.gpu_util import to_dev

pytestmark = pytest.mark.gpu


def _inputs(rows, vocab, dtype, seed, gpu):
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal((rows, vocab)) * 3).astype(np.float32)
    xd = to_dev(x, dtype, gpu)
    k = torch.from_numpy(rng.integers(1, 1025, rows).astype(np.int32)).to(gpu)
    p = torch.from_numpy(rng.uniform(0.7, 1.0, rows).astype(np.float32)).to(gpu)
    t = torch.from_numpy(rng.uniform(0.5, 1.5, rows).astype(np.float32)).to(gpu)
    key = torch.tensor([0, 1234 + seed], dtype=torch.int64).to(torch.int32).to(gpu)
    return xd, k, p, t, key


def _both(xd, k, p, t, key, dim0_offset=0):
    from tallax_amd import _lib
    rows, vocab = xd.shape
    dt = _lib.dtype_code(xd)
    s = _lib.stream_of(xd)
    need = _lib.LIB.tallax_sample_workspace_size(rows, vocab, dt)
    ws = torch.empty(max(need, 1), dtype=torch.uint8, device=xd.device)
    want = torch.full((rows,), -7, dtype=torch.int32, device=xd.device)
    got = torch.full((rows,), -9, dtype=torch.int32, device=xd.device)
    _lib.check(_lib.LIB.tallax_fused_topk_topp_sample(
        xd.data_ptr(), dt, rows, vocab, k.data_ptr(), p.data_ptr(), t.data_ptr(), key.data_ptr(), dim0_offset,
        -1e12, want.data_ptr(), ws.data_ptr(), ws.numel(), s), "sample")
    _lib.check(_lib.LIB.tallax_fused_topk_topp_sample_noalloc(
        xd.data_ptr(), dt, rows, vocab, k.data_ptr(), p.data_ptr(), t.data_ptr(), key.data_ptr(), dim0_offset,
        -1e12, got.data_ptr(), s), "sample_noalloc")
    torch.cuda.synchronize()
    return need, got.cpu().numpy(), want.cpu().numpy()


@pytest.mark.parametrize("first,second", [
    ((64, 200000, "bf16"), (16, 170000, "bf16")),     # segmented, then a smaller segmented input
    ((128, 151936, "f32"), (8, 100000, "f32")),       # config-3 width f32 (8 segments per row)
    ((256, 128256, "bf16"), (32, 100000, "f32")),     # whole rows (no scratch), then segmented
])
def test_noalloc_matches_workspace_entry(gpu, first, second):
    for n, (rows, vocab, dtype) in enumerate((first, second)):
        print(f"noalloc sampler call {n}: [{rows},{vocab}] {dtype}", flush=True)
        xd, k, p, t, key = _inputs(rows, vocab, dtype, rows + n, gpu)
        need, got, want = _both(xd, k, p, t, key, dim0_offset=3 * n)
        assert (want >= 0).all() and (want < vocab).all()
        assert np.array_equal(got, want), (rows, vocab, dtype, need)


def test_noalloc_rejects_inputs_beyond_its_scratch(gpu):
    from tallax_amd import _lib
    rows, vocab = 2048, 151936          # 2048 x 10 segments x 1 KiB = 20 MiB > 16 MiB
    dt = _lib.F32
    assert _lib.LIB.tallax_sample_workspace_size(rows, vocab, dt) > 16 << 20
    x = torch.empty((rows, vocab), dtype=torch.float32, device=gpu)
    out = torch.empty(rows, dtype=torch.int32, device=gpu)
    st = _lib.LIB.tallax_fused_topk_topp_sample_noalloc(x.data_ptr(), dt, rows, vocab, out.data_ptr(),
                                                        out.data_ptr(), out.data_ptr(), out.data_ptr(), 0, -1e12,
                                                        out.data_ptr(), _lib.stream_of(x))
    assert st == _lib.UNSUPPORTED and b"scratch" in _lib.LIB.tallax_last_error()
