"""GPU parity of the wide-candidate sampler (sampling.sample(..., max_k=K),
K <= 1024, beyond the reference's clamp at 128) and of its candidate lists
(sampling.wide_top_k), through the C ABI, against the oracle on identical
seeded inputs: candidate values and columns bit-exact, tokens exact."""
import numpy as np
import pytest
import torch

from oracle import tallax_oracle as O
from tests.gpu_util import bits, host_values, to_dev
from tests.test_gpu_select import _make, _sampler_inputs

pytestmark = pytest.mark.gpu


def _log(msg):
    print(msg, flush=True)


WIDE_TOPK_CASES = [
    (8, 32000, 1024, "bf16", "normal"),
    (8, 32000, 1024, "f32", "normal"),
    (4, 128256, 1024, "bf16", "normal"),
    (4, 32001, 129, "f32", "ints"),        # odd row length: element loads, heavy ties
    (4, 32001, 1000, "bf16", "ints"),
    (3, 5000, 1, "f32", "normal"),
    (3, 1024, 1024, "f32", "normal"),      # K == vocab
    (4, 20000, 700, "f32", "special"),     # NaN, -inf, -0, finfo.min, a row of NaN
    (4, 20000, 700, "bf16", "special"),
    (2, 128256, 1024, "bf16", "const"),
    (2, 50000, 1024, "f32", "masked5"),    # fewer eligible values than K
    (2, 50000, 1024, "f32", "tieblock"),
    (2, 50000, 512, "bf16", "nan_heavy"),
    (2, 40000, 300, "f32", "sorted_asc"),
    (3, 40000, 1024, "f32", "outlier"),    # K-th value far below the maximum: the whole-row digit passes
    (3, 40000, 1024, "bf16", "outlier"),
    (2, 6000, 1024, "bf16", "normal"),     # fewer than K threads hold an element
    (4, 151936, 1024, "bf16", "normal"),   # one read at 19 vectors per thread
    (3, 76000, 1024, "f32", "outlier"),
    (2, 200000, 1024, "bf16", "normal"),   # too long for the registers: the radix select path
]


def _make_wide(rows, cols, kind, seed):
    if kind == "outlier":
        x = _make(rows, cols, "normal", seed)
        x[:, 17] = 1e30
        x[1:, 40] = -1e30
        return x
    return _make(rows, cols, kind, seed)


@pytest.mark.parametrize("rows,cols,k,dtype,kind", WIDE_TOPK_CASES)
def test_wide_top_k_parity(gpu, rows, cols, k, dtype, kind):
    from tallax_amd import sampling
    _log(f"wide_top_k rows={rows} cols={cols} k={k} dtype={dtype} kind={kind}")
    x = _make_wide(rows, cols, kind, seed=cols + k)
    xd = to_dev(x, dtype, gpu)
    vals, idx = sampling.wide_top_k(xd, k)
    torch.cuda.synchronize()
    wv, wi = O.top_k(host_values(x, dtype), k, dtype)
    assert np.array_equal(idx.cpu().numpy(), wi)
    assert np.array_equal(bits(vals.cpu().numpy()), bits(wv))


@pytest.mark.parametrize("rows,vocab,dtype,max_k", [(256, 128256, "bf16", 1024), (64, 32000, "f32", 1024),
                                                    (32, 32001, "bf16", 300), (16, 4096, "f32", 777),
                                                    (64, 151936, "bf16", 1024)])
def test_wide_sampler_parity(gpu, rows, vocab, dtype, max_k):
    from tallax_amd import sampling
    _log(f"sample max_k={max_k} rows={rows} vocab={vocab} dtype={dtype}")
    x, temp, topk, topp = _sampler_inputs(rows, vocab, seed=vocab + max_k)
    temp[::17] = 1e-6      # greedy rows
    topk[1::13] = 1        # top-1 rows
    topp[2::11] = 1.0      # cumsum may stay below p: threshold 0
    x[3, :] = 0.25         # a constant row
    meta = sampling.SamplingMetadata(torch.from_numpy(topk), torch.from_numpy(topp), torch.from_numpy(temp))
    key = torch.tensor([11, 2024], dtype=torch.int32, device=gpu)
    got = sampling.sample(key, to_dev(x, dtype, gpu), meta, dim0_offset=3, max_k=max_k)
    torch.cuda.synchronize()
    want = O.sample((11, 2024), host_values(x, dtype), topk, topp, temp, dtype=dtype, dim0_offset=3,
                    max_k=max_k)
    assert np.array_equal(got.cpu().numpy(), want)


def test_wide_sampler_reduces_to_the_fused_sampler(gpu):
    """At config 4's shape with every k <= 128 the wide kernel (K = 1024) and
    the reference-width fused kernel draw the same tokens."""
    from tallax_amd import sampling
    x, temp, topk, topp = _sampler_inputs(256, 128256, seed=5)
    topk = np.minimum(topk, 128).astype(np.int32)
    meta = sampling.SamplingMetadata(torch.from_numpy(topk), torch.from_numpy(topp), torch.from_numpy(temp))
    xd = to_dev(x, "bf16", gpu)
    key = torch.tensor([0, 77], dtype=torch.int32, device=gpu)
    wide = sampling.sample(key, xd, meta, max_k=1024)
    ref = sampling.sample(key, xd, meta)
    torch.cuda.synchronize()
    assert np.array_equal(wide.cpu().numpy(), ref.cpu().numpy())
