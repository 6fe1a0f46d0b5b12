#!/usr/bin/env python3
"""Benchmark of the tallax MI355X hot path (one GPU).

Default workload (BASELINE.json metric / config 4): the fused top-k/top-p
sampler (`tallax_amd.sampling.sample`, one HIP kernel) on bf16 logits
[256, 128256] ~ N(0, sigma=3), per-row temperature U[0.5,1.5), top_k
uniform in [1, 1024], top_p U[0.7,1.0), threefry key data (0, 1234).
A "step" samples one token for each of the 256 rows.

Timing: inputs are resident in HBM before the timed region; the step rotates
over `--nbuf` distinct logits buffers (6 x 65.7 MB > the 256 MB MALL) so
every step streams its logits from HBM.  Whole-job time is bracketed by
torch.cuda.synchronize(); the kernel's own average duration is measured with
HIP events recorded on the stream the kernel is launched on.  One JSON line
is printed.

--config topk_c3 / topk_c1 time exact top-k (configs 3 and 1) instead;
--config copy times torch's device copy of 256 MiB (the counter calibration).
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_HBM_GBS = 8000.0  # MI355X HBM3E peak, GB/s


COPY_BYTES = 256 << 20  # calibration copy: 256 MiB read + 256 MiB written per launch


def _copy_rate(torch, dev, stream, steps, warmup):
    """Read+write GB/s of torch's device copy over COPY_BYTES (the calibration
    kernel for the FETCH_SIZE / WRITE_SIZE counters and a measured peak)."""
    n = COPY_BYTES // 4
    bufs = [torch.empty(n, dtype=torch.float32, device=dev) for _ in range(3)]
    for b in bufs:
        b.fill_(1.0)
    for s in range(warmup):
        bufs[(s + 1) % 3].copy_(bufs[s % 3])
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    e0.record(stream)
    for s in range(steps):
        bufs[(s + 1) % 3].copy_(bufs[s % 3])
    e1.record(stream)
    torch.cuda.synchronize()
    us = e0.elapsed_time(e1) * 1e3 / steps
    return 2 * COPY_BYTES / (us * 1e-6) / 1e9, us


def _measured_traffic(config):
    """HBM bytes per launch measured with rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE
    (scaled by the copy calibration), as recorded in profiles/*.md lines
    `traffic_bytes_per_launch[<config>] = <bytes>`; None if absent."""
    import glob
    import re
    pat = re.compile(r"traffic_bytes_per_launch\[" + re.escape(config) + r"\]\s*=\s*([0-9]+)")
    for f in sorted(glob.glob(os.path.join(ROOT, "profiles", "*.md"))):
        m = pat.search(open(f).read())
        if m:
            return int(m.group(1))
    return None


def _parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--config", default="sampler", choices=["sampler", "topk_c3", "topk_c1", "copy"])
    ap.add_argument("--nbuf", type=int, default=6)
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-parity", action="store_true")
    return ap.parse_args()


def main() -> int:
    args = _parse()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (--gpus {args.gpus} requested); "
              "the sort/select/sample path is single-GPU here -- see DESIGN.md for how it shards.",
              file=sys.stderr)
        return 2

    import numpy as np
    import torch

    from tallax_amd import _lib

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    stream = torch.cuda.current_stream(dev)
    s_handle = stream.cuda_stream
    gen = torch.Generator(device=dev)
    gen.manual_seed(4)

    if args.config == "copy":
        gbs, us = _copy_rate(torch, dev, stream, args.steps, args.warmup)
        print(json.dumps({"metric": "device copy GB/s (read + write), calibration", "value": gbs,
                          "unit": "GB/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
                          "ms_per_step": us / 1e3, "higher_is_better": True, "scaling": "weak",
                          "vs_baseline": None, "dtype": "f32", "data": "synthetic",
                          "config": {"workload": f"torch copy_ of {COPY_BYTES} bytes (f32)"}}), flush=True)
        return 0

    if args.config == "sampler":
        rows, cols, dt_name, sigma = 256, 128256, "bf16", 3.0
        tdt = torch.bfloat16
        rng = np.random.default_rng(5)
        temp = rng.uniform(0.5, 1.5, rows).astype(np.float32)
        topk = rng.integers(1, 1025, rows).astype(np.int32)
        topp = rng.uniform(0.7, 1.0, rows).astype(np.float32)
        d_temp = torch.from_numpy(temp).to(dev)
        d_topk = torch.from_numpy(topk).to(dev)
        d_topp = torch.from_numpy(topp).to(dev)
        key = (0, 1234)
        d_key = torch.tensor(key, dtype=torch.int32, device=dev)
        out = torch.empty(rows, dtype=torch.int32, device=dev)
        need = _lib.LIB.tallax_sample_workspace_size(rows, cols, _lib.BF16)
        ws = torch.zeros(max(need, 1), dtype=torch.uint8, device=dev)
        alg_bytes = rows * cols * 2 + rows * 12 + 8 + rows * 4
        workload = ("fused top-k/top-p/temperature/Gumbel sampler (sampling.sample): bf16 logits "
                    "[256,128256] ~ N(0,3), top_k U{1..1024} (clamped to 128), top_p U[0.7,1), "
                    "T U[0.5,1.5), threefry key (0,1234)")
        kernel_name = _lib.select_plan(rows, cols, _lib.BF16)["kernel"].replace("SAMPLE", "true")
        bufs = [(torch.randn((rows, cols), generator=gen, device=dev) * sigma).to(tdt) for _ in range(args.nbuf)]

        def launch(x):
            _lib.check(_lib.LIB.tallax_fused_topk_topp_sample(
                x.data_ptr(), _lib.BF16, rows, cols, d_topk.data_ptr(), d_topp.data_ptr(), d_temp.data_ptr(),
                d_key.data_ptr(), 0, -1e12, out.data_ptr(), ws.data_ptr(), ws.numel(), s_handle), "sample")
    else:
        if args.config == "topk_c3":
            rows, cols, k = 128, 151936, 50
            workload = ("exact top-k (tax.top_k) k=50: f32 [128,151936] ~ N(0, sigma=2) + 32 spikes/row at 8.0")
        else:
            rows, cols, k = 8, 32768, 64
            workload = "exact top-k (tax.top_k) k=64: f32 [8,32768] ~ N(0,1)"
        dt_name, tdt = "f32", torch.float32
        kernel_name = _lib.select_plan(rows, cols, _lib.F32)["kernel"].replace("SAMPLE", "false")
        need = _lib.LIB.tallax_topk_workspace_size(rows, cols, k, _lib.F32)
        ws = torch.zeros(max(need, 1), dtype=torch.uint8, device=dev)
        vals = torch.empty((rows, k), dtype=tdt, device=dev)
        idx = torch.empty((rows, k), dtype=torch.int32, device=dev)
        alg_bytes = rows * cols * 4 + rows * k * 8
        bufs = []
        for b in range(args.nbuf):
            x = torch.randn((rows, cols), generator=gen, device=dev) * (2.0 if args.config == "topk_c3" else 1.0)
            if args.config == "topk_c3":
                sp = torch.rand((rows, cols), generator=gen, device=dev).argsort(dim=1)[:, :32]
                x.scatter_(1, sp, 8.0)
            bufs.append(x.contiguous())

        def launch(x):
            _lib.check(_lib.LIB.tallax_topk(x.data_ptr(), _lib.F32, rows, cols, k, vals.data_ptr(),
                                            idx.data_ptr(), ws.data_ptr(), ws.numel(), s_handle), "top_k")
    torch.cuda.synchronize()

    # ---- parity of the benchmarked kernel on buffer 0 (outside the timed region)
    parity = None
    host0 = None
    if not args.no_parity or not args.no_cpu_baseline:
        from oracle import tallax_oracle as O
        if tdt == torch.bfloat16:
            host0 = O.bf16_bits_to_f32(bufs[0].view(torch.int16).cpu().numpy().view(np.uint16))
        else:
            host0 = bufs[0].cpu().numpy()
    if not args.no_parity:
        launch(bufs[0])
        torch.cuda.synchronize()
        if args.config == "sampler":
            want = O.sample(key, host0, topk, topp, temp, dtype="bf16")
            parity = bool(np.array_equal(out.cpu().numpy(), want))
        else:
            ov, oi = O.top_k(host0, k)
            parity = bool(np.array_equal(idx.cpu().numpy(), oi))
        print(f"bench: parity of {args.config} vs oracle on buffer 0: {parity}", file=sys.stderr, flush=True)

    # ---- warmup
    for s in range(args.warmup):
        launch(bufs[s % len(bufs)])
    torch.cuda.synchronize()

    # ---- whole-job timing
    t0 = time.perf_counter()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for s in range(args.steps):
        launch(bufs[s % len(bufs)])
    e1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    gpu_ms = e0.elapsed_time(e1)
    total_s = max(wall, gpu_ms / 1e3)
    ms_per_step = total_s * 1e3 / args.steps

    # ---- kernel duration: events around each launch on the launch stream
    n_ev = min(args.steps, 200)
    starts = [torch.cuda.Event(enable_timing=True) for _ in range(n_ev)]
    ends = [torch.cuda.Event(enable_timing=True) for _ in range(n_ev)]
    for s in range(n_ev):
        starts[s].record(stream)
        launch(bufs[s % len(bufs)])
        ends[s].record(stream)
    torch.cuda.synchronize()
    durs_us = sorted(a.elapsed_time(b) * 1e3 for a, b in zip(starts, ends))
    # Average launch duration: HIP events on the launch stream around the K
    # back-to-back launches of the timed region (per-launch event pairs add
    # their own packets to every launch, so they are reported separately).
    kern_us = gpu_ms * 1e3 / args.steps
    achieved = alg_bytes / (kern_us * 1e-6) / 1e9

    # ---- CPU baseline: the numpy oracle on a bounded sample of the same workload
    cpu = None
    if not args.no_cpu_baseline:
        rows_done = 0
        t_cpu = 0.0
        batch = 16
        r0 = 0
        while t_cpu < args.cpu_seconds:
            sl = slice(r0, r0 + batch)
            t = time.perf_counter()
            if args.config == "sampler":
                O.sample(key, host0[sl], topk[sl], topp[sl], temp[sl], dtype="bf16", dim0_offset=r0)
            else:
                O.top_k(host0[sl], k)
            t_cpu += time.perf_counter() - t
            rows_done += host0[sl].shape[0]
            r0 = (r0 + batch) % rows
        cpu = {"value": rows_done / t_cpu, "unit": "rows/s", "cores": 1, "kind": "port",
               "sample": f"{rows_done} rows ({batch}-row batches) of the same {dt_name} [{rows},{cols}] "
                         f"workload through the numpy oracle (oracle/tallax_oracle.py), single thread, "
                         f"{t_cpu:.1f} s"}

    copy_gbs, _ = _copy_rate(torch, dev, stream, 10, 3)
    rows_per_s = rows * args.steps / total_s
    rec = {
        "metric": "rows/s + achieved HBM GB/s (% peak): fused top-k/top-p @256x128256 bf16"
                  if args.config == "sampler" else f"rows/s + achieved HBM GB/s (% peak): {args.config}",
        "value": rows_per_s,
        "unit": "rows/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16" if dt_name == "bf16" else "f32",
        "data": f"synthetic (torch.randn on device, seed 4; {args.nbuf} rotating input buffers)",
        "config": {"workload": workload, "rows": rows, "cols": cols, "parallelism": "single GPU"},
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": PEAK_HBM_GBS, "unit": "GB/s",
                     "frac": achieved / PEAK_HBM_GBS, "traffic": _measured_traffic(args.config),
                     "measured_copy_GBs": copy_gbs, "frac_of_copy": achieved / copy_gbs,
                     "kernel": kernel_name, "kernel_avg_us": kern_us,
                     "event_pair_median_us": durs_us[len(durs_us) // 2],
                     "algorithmic_bytes_per_launch": alg_bytes},
        "cpu_baseline": cpu,
        "parity_vs_oracle": parity,
        "wall_ms_per_step": wall * 1e3 / args.steps,
        "gpu_event_ms_per_step": gpu_ms / args.steps,
    }
    print(json.dumps(rec), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
