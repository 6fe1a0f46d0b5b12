"""Host logic of bench.py (no GPU): the per-launch HBM traffic computed from
rocprofv3 --pmc passes, with the profiler pass replaced by fixed counter
values, and the single-GPU guard."""
import subprocess
import sys

import pytest

import bench


def _fake_pass(counter, config, extras, outdir, timeout):
    """Counter values as rocprofv3 lists them for one pass: FETCH_SIZE reports
    half of the bytes read (the copy reads COPY_BYTES = 262144 KiB and shows
    131072), WRITE_SIZE all of the bytes written."""
    launches = bench.PMC_WARMUP + bench.PMC_STEPS
    c5 = bench.PMC_WARMUP + bench._extra_steps("prefill_c5", bench.PMC_STEPS)
    if counter == "FETCH_SIZE":
        return {
            bench.COPY_KERNEL: [131072.0] * 13 + [1.0, 2.0],          # the calibration + small torch copies
            "void tx::stream_select_kernel<1, 16, true, false>(tx::SelArgs)": [32000.0] * (launches - 1) + [32100.0],
            "tx::seg_select_kernel<0, 19, 256, false>": [38000.0] * launches,
            "tx::seg_merge64_kernel<0>": [300.0] * launches,
            "tx::softmax_topk_kernel<true>": [500000.0] * c5,
            "tx::radix_sort_rows_kernel<8>": [1000.0] * launches,
            "tx::gather_row_lds_kernel<unsigned int>": [4000.0] * launches,
            "at::native::normal_kernel": [99999.0] * 7,               # input generation: not counted
        }
    return {
        bench.COPY_KERNEL: [262144.0] * 13 + [1.0],
        "tx::stream_select_kernel<1, 16, true, false>": [8.0] * launches,
        "tx::seg_select_kernel<0, 19, 256, false>": [1024.0] * launches,
        "tx::seg_merge64_kernel<0>": [56.0] * launches,
        "tx::softmax_topk_kernel<true>": [24000.0] * c5,
        "tx::radix_sort_rows_kernel<8>": [6144.0] * launches,
        "tx::gather_row_lds_kernel<unsigned int>": [4096.0] * launches,
    }


def test_live_traffic_arithmetic(monkeypatch):
    monkeypatch.setattr(bench, "_pmc_pass", _fake_pass)
    per, scale = bench._live_traffic("sampler", extras=True)
    assert scale == {"FETCH_SIZE": 2.0, "WRITE_SIZE": 1.0}
    # medians per dispatch x dispatches per launch, reads doubled
    assert per["sampler"] == (32000 * 2 + 8) * 1024
    assert per["topk_c3"] == ((38000 + 300) * 2 + 1024 + 56) * 1024
    assert per["prefill_c5"] == (500000 * 2 + 24000) * 1024
    assert per["sort_c2"] == ((1000 + 4000) * 2 + 6144 + 4096) * 1024


def test_live_traffic_without_extras_counts_main_config_only(monkeypatch):
    monkeypatch.setattr(bench, "_pmc_pass", _fake_pass)
    per, _ = bench._live_traffic("sampler", extras=False)
    assert set(per) == {"sampler"}


def test_live_traffic_rejects_a_pass_without_the_calibration(monkeypatch):
    def no_copy(counter, config, extras, outdir, timeout):
        v = _fake_pass(counter, config, extras, outdir, timeout)
        del v[bench.COPY_KERNEL]
        return v
    monkeypatch.setattr(bench, "_pmc_pass", no_copy)
    with pytest.raises(RuntimeError, match="no __amd_rocclr_copyBuffer"):
        bench._live_traffic("sampler", extras=False)


def test_live_traffic_rejects_a_pass_without_the_kernel(monkeypatch):
    def no_kernel(counter, config, extras, outdir, timeout):
        v = _fake_pass(counter, config, extras, outdir, timeout)
        return {k: x for k, x in v.items() if "stream_select" not in k}
    monkeypatch.setattr(bench, "_pmc_pass", no_kernel)
    with pytest.raises(RuntimeError, match="no dispatch of sampler"):
        bench._live_traffic("sampler", extras=False)


def test_every_config_with_a_launch_names_its_kernels():
    for c in bench.CONFIGS:
        if c not in ("copy", "read_calib"):
            assert bench.TRAFFIC_KERNELS[c]


def test_recorded_traffic_matches_profiles():
    assert bench._recorded_traffic("sampler") > 65671176
    assert bench._recorded_traffic("no_such_config") is None


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, bench.__file__, "--gpus", "2"], capture_output=True, text=True, timeout=60)
    assert r.returncode == 2 and "one GPU only" in r.stderr
