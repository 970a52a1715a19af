#!/usr/bin/env python3
"""Throughput of the MI355X token sampler on the indextts mel-code workload.

One step = one tc_sample launch over one batch of 256 rows x 8194 f32 logits
(history 1500 Zipf ids per row, repetition penalty 10, T 0.8, top-k 30,
top-p 0.8, one f64 uniform per row), with inputs already resident in HBM.
Batches rotate through a pool larger than twice the 256 MB Infinity Cache so
every step streams its logits from HBM.

Prints one JSON line: rows/s for the whole job, the roofline figure of the
sampler kernel (algorithmic bytes per launch over its average duration,
timed with HIP events on the launch stream), and the CPU baseline (the oracle
timed on this host on a bounded sample of the same workload).

    python bench.py [--gpus 1] [--steps 2000] [--warmup 200]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

HBM_PEAK_GBS = 8000.0
METRIC = "sampled rows/sec + achieved HBM GB/s (% of ~8 TB/s) at vocab 8194, batch 256"


def parse():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2000)
    ap.add_argument("--warmup", type=int, default=200)
    ap.add_argument("--workload", default="indextts-mel-256x8194")
    ap.add_argument("--pool-mb", type=int, default=640, help="rotating input pool (MB of logits)")
    ap.add_argument("--cpu-seconds", type=float, default=12.0, help="CPU baseline sample budget")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--copy-calib", action="store_true",
                    help="after the timed region, copy 256 MiB three times (calibrates rocprofv3 byte counters)")
    return ap.parse_args()


PROFILES = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles")


def measured_traffic(workload: str):
    """HBM bytes per launch of the sampler kernel, measured with rocprofv3 --pmc
    FETCH_SIZE / WRITE_SIZE and scaled by a plain copy of known size (the
    summary in profiles/traffic_<workload>.txt), or None."""
    path = os.path.join(PROFILES, f"traffic_{workload}.txt")
    if not os.path.exists(path):
        return None
    for line in open(path):
        if line.startswith("bytes_per_launch:"):
            return int(float(line.split(":", 1)[1]))
    return None


def cpu_baseline(w, batch, seconds: float):
    """The oracle (C restatement of the reference Rust sampler) on this host."""
    from oracle import oracle as O

    p = O.make_params(w.variant, temperature=w.temperature, top_k=w.top_k, top_p=w.top_p,
                      penalty=w.penalty, min_keep=w.min_keep, ras_win=w.ras_win, ras_tau=w.ras_tau)
    rows = batch.logits_f32.shape[0]
    O.sample(p, batch.logits_f32[:8], batch.hist_off[:9], batch.hist_ids, batch.uniforms[:8 * w.n_uniforms])
    done, t0 = 0, time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        O.sample(p, batch.logits_f32, batch.hist_off, batch.hist_ids, batch.uniforms, nthreads=1)
        done += rows
    dt = time.perf_counter() - t0
    return {"value": round(done / dt, 1), "unit": "rows/s", "cores": 1, "kind": "port",
            "sample": f"{done} rows of {w.name} ({done // rows} passes over one seeded batch), "
                      f"single thread, {dt:.1f} s"}


def main():
    args = parse()
    if args.gpus != 1:
        print("bench.py: this sampler runs on one GPU; multi-GPU runs are not part of this build "
              "(rows are independent: each GPU would run the same kernel on its share of the batch)",
              file=sys.stderr)
        sys.exit(2)
    import torch

    from talechime_amd import synth
    from talechime_amd.sampler import DeviceSampler, make_params

    w = synth.WORKLOADS[args.workload]
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    batch = synth.make_batch(w)
    per_batch = w.rows * w.vocab * w.logit_bytes
    n_pool = max(2, int(np.ceil(args.pool_mb * 1e6 / per_batch)))
    # pool: the seeded batch first, then batches of the same shape and distribution
    g = torch.Generator(device=dev)
    g.manual_seed(w.seed)
    logits, hists = [], []
    first = torch.from_numpy(batch.logits).to(dev)
    hoff = torch.from_numpy(batch.hist_off.view(np.int32).copy()).to(dev)
    hid0 = torch.from_numpy(batch.hist_ids.view(np.int32).copy()).to(dev)
    for i in range(n_pool):
        if i == 0:
            logits.append(first)
            hists.append(hid0)
        else:
            logits.append(torch.randn(first.shape, generator=g, device=dev, dtype=torch.float32) * w.sigma)
            hists.append(hid0[torch.randperm(hid0.numel(), generator=g, device=dev)])
    unis = [torch.from_numpy(batch.uniforms).to(dev)]
    unis += [torch.rand(batch.uniforms.size, generator=g, device=dev, dtype=torch.float64) for _ in range(n_pool - 1)]
    sampler = DeviceSampler(0, max_rows=w.rows, max_vocab=w.vocab)
    params = make_params(w.variant, temperature=w.temperature, top_k=w.top_k, top_p=w.top_p,
                         penalty=w.penalty, min_keep=w.min_keep, ras_win=w.ras_win, ras_tau=w.ras_tau)
    outs = [None] * n_pool

    def step(i):
        j = i % n_pool
        outs[j] = sampler.sample(params, logits[j], hoff, hists[j], unis[j], out=outs[j])

    stream = torch.cuda.current_stream(dev)
    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()
    # whole-job throughput: K back-to-back steps between two events
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    e0.record(stream)
    for i in range(args.steps):
        step(i)
    e1.record(stream)
    torch.cuda.synchronize()
    ms_total = e0.elapsed_time(e1)
    ms_per_step = ms_total / args.steps
    # per-launch kernel time: an event pair around each launch on the same stream
    n_k = min(args.steps, 500)
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(n_k)]
    for i in range(n_k):
        evs[i][0].record(stream)
        step(i)
        evs[i][1].record(stream)
    torch.cuda.synchronize()
    k_ms = np.array([a.elapsed_time(b) for a, b in evs])
    k_avg_us = float(k_ms.mean() * 1e3)
    k_med_us = float(np.median(k_ms) * 1e3)
    # parity spot check of the seeded batch (first pool entry) against nothing on the
    # host: the status must be clean for every row
    st = outs[0].status.cpu().numpy()
    if (st != 0).any():
        print(f"bench.py: {int((st != 0).sum())} rows returned a non-OK status", file=sys.stderr)
        sys.exit(1)
    if args.copy_calib:
        src = torch.empty(256 << 20, dtype=torch.uint8, device=dev)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
    bytes_per_row = w.algorithmic_bytes_per_row()
    bytes_per_launch = bytes_per_row * w.rows
    achieved = bytes_per_launch / (k_avg_us * 1e-6) / 1e9
    rows_per_s = w.rows / (ms_per_step * 1e-3)
    res = {
        "metric": METRIC,
        "value": round(rows_per_s, 1),
        "unit": "rows/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32" if w.dtype == "f32" else "bf16",
        "data": "synthetic (seeded N(0,4^2) logits, Zipf(1.1) histories; rotating pool)",
        "config": {"workload": w.name, "rows": w.rows, "vocab": w.vocab, "history": w.hist_len,
                   "penalty": w.penalty, "temperature": w.temperature, "top_k": w.top_k, "top_p": w.top_p,
                   "variant": "indextts", "pool_batches": n_pool, "seed": w.seed},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": measured_traffic(w.name),
                     "kernel_avg_us": round(k_avg_us, 3), "kernel_median_us": round(k_med_us, 3),
                     "algorithmic_bytes_per_launch": bytes_per_launch},
    }
    if not args.no_cpu:
        res["cpu_baseline"] = cpu_baseline(w, batch, args.cpu_seconds)
    sampler.close()
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
