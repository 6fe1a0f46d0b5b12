"""GPU: every entry point can be captured into a HIP graph (torch.cuda.CUDAGraph
on ROCm) and replayed.  The library launches only on the caller's stream,
allocates nothing and records no memset nodes, so a captured sequence must
give, on every replay, exactly what eager calls give on the same inputs.

Each replay follows new input values written eagerly into the captured input
buffers, and is checked bit for bit against eager calls made after it (with
synchronisations in between), several times in a row.  Every entry point is
deterministic, including the config-5 softmax sums (per-batch sums merged in
batch order), so bit equality is the bar."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _log(msg):
    print(msg, flush=True)


def _fill(gen, bufs):
    """New seeded contents for the captured input buffers (eager work between replays)."""
    with torch.no_grad():
        bufs["sample_x"].copy_((torch.randn(bufs["sample_x"].shape, generator=gen, device=gen.device) * 3)
                               .to(torch.bfloat16))
        bufs["topk_x"].copy_(torch.randn(bufs["topk_x"].shape, generator=gen, device=gen.device) * 2)
        bufs["sort_x"].copy_(torch.round(torch.randn(bufs["sort_x"].shape, generator=gen, device=gen.device) * 8) / 8)
        bufs["pf_x"].copy_(torch.randn(bufs["pf_x"].shape, generator=gen, device=gen.device) * 2)
        bufs["cs_x"].copy_(torch.randn(bufs["cs_x"].shape, generator=gen, device=gen.device))


def _run_all(b):
    from tallax_amd import prefill, sampling, tax, tumpy
    meta = sampling.SamplingMetadata(b["top_k"], b["top_p"], b["temp"])
    out = {}
    out["tokens"] = sampling.sample(b["key"], b["sample_x"], meta)
    out["topk_v"], out["topk_i"] = tax.top_k(b["topk_x"], k=50)
    out["dyn"] = tax.top_dynamic_k(b["topk_x"], k=50, max_k=50)
    out["sort_k"], out["sort_p"] = tax.sort(b["sort_x"], num_keys=1, is_stable=True, return_argsort=True,
                                            descending=True)
    out["gather"] = tumpy.take_along_axis(b["sort_x"], out["sort_p"], 1)
    out["pf"] = prefill.softmax_topk_cumsum(b["pf_x"], k=256, p=0.9)
    out["cumsum"] = tax.cumsum(b["cs_x"], axis=1)
    return out


def _flat(out):
    res = []
    for k in sorted(out):
        v = out[k]
        res += [t for t in v] if isinstance(v, tuple) else [v]
    return res


def _same(a: torch.Tensor, b: torch.Tensor) -> bool:
    a, b = a.cpu(), b.cpu()
    if a.dtype in (torch.float32, torch.bfloat16):
        a = a.view(torch.int32) if a.dtype == torch.float32 else a.view(torch.int16)
        b = b.view(torch.int32) if b.dtype == torch.float32 else b.view(torch.int16)
    return bool(torch.equal(a, b))


def test_graph_capture_and_replays(gpu):
    rng = np.random.default_rng(77)
    rows = 128
    b = {
        "sample_x": torch.empty((rows, 32000), dtype=torch.bfloat16, device=gpu),
        "topk_x": torch.empty((16, 100000), dtype=torch.float32, device=gpu),  # segmented + merge kernel
        "sort_x": torch.empty((3, 40000), dtype=torch.float32, device=gpu),    # wide rows: chunk + merge passes
        "pf_x": torch.empty((8, 30000), dtype=torch.float32, device=gpu),
        "cs_x": torch.empty((8, 3000), dtype=torch.float32, device=gpu),
        "top_k": torch.from_numpy(rng.integers(1, 1025, rows).astype(np.int32)).to(gpu),
        "top_p": torch.from_numpy(rng.uniform(0.7, 1.0, rows).astype(np.float32)).to(gpu),
        "temp": torch.from_numpy(rng.uniform(0.5, 1.5, rows).astype(np.float32)).to(gpu),
        "key": torch.tensor([0, 1234], dtype=torch.int32, device=gpu),
    }
    gen = torch.Generator(device=gpu)
    gen.manual_seed(1)
    _fill(gen, b)
    # eager first: raises the dynamic-LDS limits and sizes the cached workspace
    _run_all(b)
    torch.cuda.synchronize()
    side = torch.cuda.Stream(device=gpu)  # default priority
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        _run_all(b)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    _log("capturing every entry point into one graph")
    with torch.cuda.graph(g):
        captured = _flat(_run_all(b))
    torch.cuda.synchronize()
    for rep in range(4):
        _fill(gen, b)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        got = [t.clone() for t in captured]
        want = _flat(_run_all(b))
        torch.cuda.synchronize()
        _log(f"replay {rep}: {len(got)} outputs")
        for i, (x, y) in enumerate(zip(got, want)):
            assert _same(x, y), f"replay {rep}: output {i} differs from eager"
