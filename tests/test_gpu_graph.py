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
        bufs["na_x"].copy_((torch.randn(bufs["na_x"].shape, generator=gen, device=gen.device) * 3)
                           .to(torch.bfloat16))


def _noalloc(b, x):
    """tallax_fused_topk_topp_sample_noalloc through the C ABI (static device
    scratch, no workspace): returns (status, tokens)."""
    from tallax_amd import _lib
    rows, vocab = x.shape
    out = torch.full((rows,), -3, dtype=torch.int32, device=x.device)
    st = _lib.LIB.tallax_fused_topk_topp_sample_noalloc(
        x.data_ptr(), _lib.dtype_code(x), rows, vocab, b["na_k"].data_ptr(), b["na_p"].data_ptr(),
        b["na_t"].data_ptr(), b["key"].data_ptr(), 0, -1e12, out.data_ptr(), _lib.stream_of(x))
    return st, out


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
    st, out["noalloc"] = _noalloc(b, b["na_x"])   # [64, 200000] bf16: two whole-row parts per row, lists in the static scratch
    assert st == 0
    return out


def _workspace_tokens(b):
    """The workspace entry point (tallax_fused_topk_topp_sample) on the noalloc input."""
    from tallax_amd import sampling
    meta = sampling.SamplingMetadata(b["na_k"], b["na_p"], b["na_t"])
    return sampling.sample(b["key"], b["na_x"], meta)


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


def _buffers(gpu, rng):
    rows, na_rows = 128, 64
    return {
        "sample_x": torch.empty((rows, 32000), dtype=torch.bfloat16, device=gpu),
        "topk_x": torch.empty((16, 100000), dtype=torch.float32, device=gpu),  # segmented + merge kernel
        "sort_x": torch.empty((3, 40000), dtype=torch.float32, device=gpu),    # wide rows: chunk + merge passes
        "pf_x": torch.empty((8, 30000), dtype=torch.float32, device=gpu),
        "cs_x": torch.empty((8, 3000), dtype=torch.float32, device=gpu),
        "top_k": torch.from_numpy(rng.integers(1, 1025, rows).astype(np.int32)).to(gpu),
        "top_p": torch.from_numpy(rng.uniform(0.7, 1.0, rows).astype(np.float32)).to(gpu),
        "temp": torch.from_numpy(rng.uniform(0.5, 1.5, rows).astype(np.float32)).to(gpu),
        "key": torch.tensor([0, 1234], dtype=torch.int32, device=gpu),
        "na_x": torch.empty((na_rows, 200000), dtype=torch.bfloat16, device=gpu),
        "na_k": torch.from_numpy(rng.integers(1, 1025, na_rows).astype(np.int32)).to(gpu),
        "na_p": torch.from_numpy(rng.uniform(0.7, 1.0, na_rows).astype(np.float32)).to(gpu),
        "na_t": torch.from_numpy(rng.uniform(0.5, 1.5, na_rows).astype(np.float32)).to(gpu),
    }


def test_noalloc_first_call_under_capture(gpu):
    """A device's first no-allocation call made while the stream captures:
    the scratch address is not looked up under capture, so the call returns
    TALLAX_UNSUPPORTED with a message and the capture stays valid (the rest
    of the captured work replays correctly).  After one uncaptured call the
    same call captures, and its replays match the workspace entry point.
    This file runs before tests/test_zz_no_alloc.py, so the captured call is
    the process's first; if an earlier noalloc call already looked the address
    up, the captured call succeeds and only the replay checks apply."""
    from tallax_amd import _lib
    rng = np.random.default_rng(5)
    b = _buffers(gpu, rng)
    gen = torch.Generator(device=gpu)
    gen.manual_seed(2)
    _fill(gen, b)
    _workspace_tokens(b)       # workspace entry point warm (its shared workspace sized outside capture)
    torch.cuda.synchronize()
    y = torch.zeros(1000, device=gpu)
    x = torch.randn(1000, device=gpu)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        y.copy_(x * 2)
        st, tok = _noalloc(b, b["na_x"])
    torch.cuda.synchronize()
    msg = _lib.LIB.tallax_last_error()
    _log(f"first noalloc call under capture: status {st} ({msg.decode()})")
    g.replay()
    torch.cuda.synchronize()
    assert torch.equal(y, x * 2)
    if st != 0:
        assert st == _lib.UNSUPPORTED and b"capture" in msg
        st2, tok2 = _noalloc(b, b["na_x"])       # eager: looks the address up
        torch.cuda.synchronize()
        assert st2 == 0 and torch.equal(tok2, _workspace_tokens(b))
        g2 = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g2):
            st3, tok = _noalloc(b, b["na_x"])
        assert st3 == 0
        g = g2
    for rep in range(3):
        _fill(gen, b)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        got = tok.clone()
        want = _workspace_tokens(b)
        torch.cuda.synchronize()
        assert torch.equal(got, want), f"replay {rep}"


def test_graph_capture_and_replays(gpu):
    rng = np.random.default_rng(77)
    b = _buffers(gpu, rng)
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
        cap = _run_all(b)
    captured = _flat(cap)
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
        # the captured noalloc tokens against the eager workspace entry point on the same input
        na = got[[i for i, t in enumerate(captured) if t is cap["noalloc"]][0]]
        assert torch.equal(na, _workspace_tokens(b)), f"replay {rep}: noalloc differs from the workspace entry"
