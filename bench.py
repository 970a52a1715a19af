#!/usr/bin/env python3
"""Throughput of the MI355X token sampler on the indextts mel-code workload
(--workload selects one of the other seeded configurations instead).

One step = one tc_sample launch over one batch of 256 rows x 8194 f32 logits
(history 1500 Zipf ids per row, repetition penalty 10, T 0.8, top-k 30,
top-p 0.8, one f64 uniform per row), with inputs already resident in HBM.
Batches rotate through a pool larger than twice the 256 MB Infinity Cache so
every step streams its logits from HBM.

The timed region is exactly --steps launches, captured in HIP graphs (one
launch per pool batch) and replayed, so the launches run back to back on the
GPU (a launch from Python costs a few tens of microseconds of host time; that
host-inclusive rate is reported under "timing").  Prints one JSON line:
rows/s for the whole job, the roofline figure of the sampler kernel
(algorithmic bytes per launch over its average duration, timed with HIP
events on the launch stream), "parity" (the device's ids on pool batches
against the oracle's, with the tie and unsupported rows counted) and the CPU
baseline (the oracle timed on this host, one thread and row-parallel, on a
bounded sample of the same workload).

    python bench.py [--gpus 1] [--steps 2000] [--warmup 200]
    python bench.py --parity 4      # boundary-row counts of every workload
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
    ap.add_argument("--parity-batches", type=int, default=8,
                    help="pool batches whose ids are compared with the oracle after the timed region")
    ap.add_argument("--parity", type=int, default=0, metavar="N",
                    help="instead of timing: compare N seeded batches of every workload with the oracle "
                         "and print the boundary-row counts")
    ap.add_argument("--beam", type=int, default=0, metavar="B",
                    help="time the indextts beam-sample step over B elements x 3 beams instead")
    ap.add_argument("--head", type=int, default=0, metavar="R",
                    help="time the indextts LM head (1280 -> 8194, bf16 weights) for R rows, alone and fused "
                         "with the sampler, instead")
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


def host_cpus():
    """(threads to use, CPUs this process may run on, nproc, CPU model)."""
    nproc = os.cpu_count() or 1
    try:
        avail = len(os.sched_getaffinity(0))
    except AttributeError:  # pragma: no cover
        avail = nproc
    model = "unknown"
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:  # pragma: no cover
        pass
    # one GPU's share of a shared host is 16 CPUs, whatever nproc reports
    return max(1, min(avail, 16)), avail, nproc, model


def _oracle_rate(O, p, w, batch, seconds: float, nthreads: int):
    rows = batch.logits_f32.shape[0]
    done, t0 = 0, time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        O.sample(p, batch.logits_f32, batch.hist_off, batch.hist_ids, batch.uniforms, nthreads=nthreads)
        done += rows
    return done, time.perf_counter() - t0


def cpu_baseline(w, batch, seconds: float):
    """The oracle (C restatement of the reference Rust sampler) on this host:
    one thread (the reference loops over rows serially) and row-parallel over
    the host's CPUs (OpenMP over rows)."""
    from oracle import oracle as O

    p = O.make_params(w.variant, temperature=w.temperature, top_k=w.top_k, top_p=w.top_p,
                      penalty=w.penalty, min_keep=w.min_keep, ras_win=w.ras_win, ras_tau=w.ras_tau)
    rows = batch.logits_f32.shape[0]
    O.sample(p, batch.logits_f32[:8], batch.hist_off[:9], batch.hist_ids, batch.uniforms[:8 * w.n_uniforms])
    threads, avail, nproc, model = host_cpus()
    d1, t1 = _oracle_rate(O, p, w, batch, seconds, 1)
    dn, tn = _oracle_rate(O, p, w, batch, seconds / 2, threads)
    return {"value": round(dn / tn, 1), "unit": "rows/s", "cores": threads, "kind": "port",
            "sample": f"{dn} rows of {w.name} ({dn // rows} passes over one seeded batch), rows split over "
                      f"{threads} threads, {tn:.1f} s",
            "single_thread": {"value": round(d1 / t1, 1), "unit": "rows/s", "cores": 1,
                              "sample": f"{d1} rows ({d1 // rows} passes), one thread, {t1:.1f} s"},
            "host": {"nproc": nproc, "affinity_cpus": avail, "cpu_model": model}}


def parity_counts(ids, st, fl, o):
    """Device outputs (production path, no verification outputs) against the
    oracle's on the same rows: the boundary rows are counted, not hidden."""
    ok = (st == 0) & (o["status"] == 0)
    tie = ((fl & 1) != 0) | ((o["flags"] & 1) != 0)
    near = (fl & 16) != 0
    diff = ok & (ids != o["ids"])
    return {"rows": int(ids.size), "both_ok": int(ok.sum()), "ids_equal": int((ok & (ids == o["ids"])).sum()),
            "status_mismatch": int((st != o["status"]).sum()), "unsupported": int((st == 7).sum()),
            "tie_cut_rows": int(tie.sum()), "near_tie_rows": int(near.sum()),
            "exact_sum_rows": int(((fl & 32) != 0).sum()),
            "ids_differ_on_tie_rows": int((diff & (tie | near)).sum()),
            "ids_differ_elsewhere": int((diff & ~(tie | near)).sum())}


def merge_counts(acc, c):
    if acc is None:
        return dict(c)
    return {k: acc[k] + c[k] for k in acc}


def pool_parity(w, logits, hists, hoff, unis, sampler, params, n_batches):
    """Pool batches sampled on the device compared with the oracle on the host."""
    import torch

    from oracle import oracle as O

    if n_batches <= 0:
        return None

    p = O.make_params(w.variant, temperature=w.temperature, top_k=w.top_k, top_p=w.top_p,
                      penalty=w.penalty, min_keep=w.min_keep, ras_win=w.ras_win, ras_tau=w.ras_tau)
    threads = host_cpus()[0]
    acc = None
    ho = hoff.cpu().numpy().view(np.uint32)
    for j in range(min(n_batches, len(logits))):
        r = sampler.sample(params, logits[j], hoff, hists[j], unis[j])
        torch.cuda.synchronize()
        x = logits[j].float().cpu().numpy()
        o = O.sample(p, x, ho, hists[j].cpu().numpy().view(np.uint32), unis[j].cpu().numpy(), nthreads=threads)
        acc = merge_counts(acc, parity_counts(r.ids.cpu().numpy().view(np.uint32), r.status.cpu().numpy(),
                                              r.flags.cpu().numpy().view(np.uint32), o))
    acc["batches"] = min(n_batches, len(logits))
    return acc


def parity_all(n_batches: int):
    """Every workload: n seeded batches on the device against the oracle."""
    import torch

    from oracle import oracle as O
    from talechime_amd import synth
    from talechime_amd.sampler import DeviceSampler, make_params

    dev = torch.device("cuda", 0)
    threads = host_cpus()[0]
    for name, w in synth.WORKLOADS.items():
        sampler = DeviceSampler(0, max_rows=w.rows, max_vocab=w.vocab)
        kw = dict(temperature=w.temperature, top_k=w.top_k, top_p=w.top_p, penalty=w.penalty,
                  min_keep=w.min_keep, ras_win=w.ras_win, ras_tau=w.ras_tau)
        params, op = make_params(w.variant, **kw), O.make_params(w.variant, **kw)
        acc = None
        for bi in range(n_batches):
            b = synth.make_batch(w, batch_index=bi)
            if w.dtype == "bf16":
                lg = torch.from_numpy(b.logits.view(np.int16).copy()).view(torch.bfloat16).to(dev)
            else:
                lg = torch.from_numpy(b.logits).to(dev)
            hid = b.hist_ids if b.hist_ids.size else np.zeros(1, np.uint32)
            r = sampler.sample(params, lg, torch.from_numpy(b.hist_off.view(np.int32).copy()).to(dev),
                               torch.from_numpy(hid.view(np.int32).copy()).to(dev),
                               torch.from_numpy(b.uniforms).to(dev))
            torch.cuda.synchronize()
            o = O.sample(op, b.logits_f32, b.hist_off, b.hist_ids, b.uniforms, nthreads=threads)
            acc = merge_counts(acc, parity_counts(r.ids.cpu().numpy().view(np.uint32), r.status.cpu().numpy(),
                                                  r.flags.cpu().numpy().view(np.uint32), o))
        sampler.close()
        acc["batches"] = n_batches
        print(json.dumps({"workload": name, **acc}), flush=True)


def beam_bench(args):
    """The indextts beam-sample step (tc_indextts_beam_step) over B elements of
    3 beams of the mel-code rows, 6 draws each, timed like the sampler step:
    a HIP graph of launches over a rotating pool, replayed."""
    import torch

    from talechime_amd import synth
    from talechime_amd.sampler import DeviceSampler, make_params

    w = synth.WORKLOADS["indextts-mel-256x8194"]
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    nb, B = 3, args.beam
    bb = synth.make_beam_batch(w, B, nb)
    rows = B * nb
    per_batch = rows * w.vocab * 4
    n_pool = min(256, max(2, int(np.ceil(args.pool_mb * 1e6 / per_batch))))
    g = torch.Generator(device=dev)
    g.manual_seed(w.seed)
    first = torch.from_numpy(bb.logits).to(dev)
    logits = [first] + [torch.randn(first.shape, generator=g, device=dev) * w.sigma for _ in range(n_pool - 1)]
    hoff = torch.from_numpy(bb.hist_off.view(np.int32).copy()).to(dev)
    hid = torch.from_numpy(bb.hist_ids.view(np.int32).copy()).to(dev)
    bs = torch.from_numpy(bb.beam_scores).to(dev)
    un = torch.from_numpy(bb.uniforms).to(dev)
    sampler = DeviceSampler(0, max_rows=rows, max_vocab=w.vocab)
    p = make_params(w.variant, temperature=w.temperature, top_k=w.top_k, top_p=w.top_p, penalty=w.penalty,
                    min_keep=w.min_keep)
    outs = [None] * n_pool

    def step(j):
        outs[j] = sampler.beam_step(p, logits[j], hoff, hid, bs, nb, un)

    for i in range(max(args.warmup, n_pool)):
        step(i % n_pool)
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream(dev)

    def capture(n):
        if n == 0:
            return None
        gr = torch.cuda.CUDAGraph()
        with torch.cuda.graph(gr):
            for j in range(n):
                step(j)
        return gr

    K = max(1, args.steps)
    full_replays, rest = divmod(K, n_pool)
    full, part = capture(n_pool), capture(rest)
    full.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(full_replays):
        full.replay()
    if part is not None:
        part.replay()
    e1.record(stream)
    torch.cuda.synchronize()
    steps = full_replays * n_pool + rest
    ms = e0.elapsed_time(e1) / steps
    st = outs[0].status.cpu().numpy()
    if (st != 0).any():
        print(f"bench.py: {int((st != 0).sum())} beam elements returned a non-OK status", file=sys.stderr)
        sys.exit(1)
    sampler.close()
    # algorithmic bytes per step: every beam row's logits and history, its beam
    # score, the element's uniforms, and the candidates written (flat u32 + f64)
    n_draws = 2 * nb
    step_bytes = rows * (w.vocab * 4 + w.hist_len * 4 + 8) + B * n_draws * (8 + 4 + 8) + B * 8
    achieved = step_bytes / (ms * 1e-3) / 1e9
    extra = {"roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                          "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None,
                          "algorithmic_bytes_per_step": step_bytes,
                          "note": "latency-bound: two launches per step (row pass, joint draws); the joint draws move a few KB"}}
    if not args.no_cpu:
        extra["cpu_baseline"] = beam_cpu_baseline(w, bb, nb, args.cpu_seconds)
    print(json.dumps({
        "metric": f"indextts beam-sample steps/sec ({B} elements x {nb} beams x {w.vocab}, 6 draws)",
        "value": round(1e3 / ms, 1), "unit": "steps/s", "n_gpus": 1, "steps": steps, "warmup": args.warmup,
        "ms_per_step": round(ms, 6), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "f32", "data": "synthetic (seeded mel-code rows, running beam scores; rotating pool)",
        "config": {"workload": f"indextts-beam-{B}x{nb}x{w.vocab}", "elements": B, "num_beams": nb,
                   "n_draws": 2 * nb, "pool_batches": n_pool},
        "timing": f"{steps} steps (row pass + joint draws each): {full_replays} replays of a HIP graph of "
                  f"{n_pool} steps" + (f" and one of {rest}" if rest else ""),
        **extra,
    }), flush=True)


def head_bench(args):
    """The LM head before the sampler (tc_lm_head) for R rows of the indextts
    mel_head (1280 -> 8194, bf16 weights, f32 bias), and the head fused with
    the mel-code sampler (tc_head_sample).  A rotating pool of weight matrices
    larger than twice the Infinity Cache keeps every launch reading HBM."""
    import torch

    from talechime_amd import synth
    from talechime_amd.sampler import DeviceSampler, make_params

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    R, dim, vocab = args.head, 1280, 8194
    wbytes = vocab * dim * 2
    n_pool = max(2, int(np.ceil(args.pool_mb * 1e6 / wbytes)))
    g = torch.Generator(device=dev)
    g.manual_seed(11)
    weights = [(torch.randn(vocab, dim, generator=g, device=dev) * 0.05).to(torch.bfloat16) for _ in range(n_pool)]
    bias = torch.randn(vocab, generator=g, device=dev) * 0.5
    hidden = [torch.randn(R, dim, generator=g, device=dev) for _ in range(n_pool)]
    logits = [torch.empty(R, vocab, device=dev) for _ in range(n_pool)]
    w = synth.WORKLOADS["indextts-mel-256x8194"]
    bt = synth.make_batch(w, rows=R)
    ho = torch.from_numpy(bt.hist_off.view(np.int32).copy()).to(dev)
    hi = torch.from_numpy(bt.hist_ids.view(np.int32).copy()).to(dev)
    un = torch.from_numpy(bt.uniforms).to(dev)
    sampler = DeviceSampler(0, max_rows=max(R, 8), max_vocab=vocab)
    params = make_params(w.variant, temperature=w.temperature, top_k=w.top_k, top_p=w.top_p, penalty=w.penalty,
                         min_keep=w.min_keep)
    stream = torch.cuda.current_stream(dev)

    def timed(step):
        for j in range(n_pool):
            step(j)
        torch.cuda.synchronize()
        full_replays, rest = divmod(max(1, args.steps), n_pool)

        def capture(n):
            if n == 0:
                return None
            gr = torch.cuda.CUDAGraph()
            with torch.cuda.graph(gr):
                for j in range(n):
                    step(j)
            return gr
        full, part = capture(n_pool), capture(rest)
        full.replay()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(full_replays):
            full.replay()
        if part is not None:
            part.replay()
        e1.record(stream)
        torch.cuda.synchronize()
        n = full_replays * n_pool + rest
        return e0.elapsed_time(e1) / n, n

    ms_head, n = timed(lambda j: sampler.lm_head(hidden[j], weights[j], bias, out=logits[j]))
    outs = [None] * n_pool

    def fused(j):
        outs[j] = sampler.head_sample(params, hidden[j], weights[j], bias, ho, hi, un, logits=logits[j])
    ms_fused, _ = timed(fused)
    st = outs[0].status.cpu().numpy()
    if (st != 0).any():
        print("bench.py: the fused head step returned a non-OK status", file=sys.stderr)
        sys.exit(1)
    step_bytes = wbytes + R * dim * 4 + vocab * 4 + R * vocab * 4
    achieved = step_bytes / (ms_head * 1e-3) / 1e9
    res = {
        "metric": f"indextts mel_head GEMV (1280 -> 8194 bf16) steps/sec, {R} rows",
        "value": round(1e3 / ms_head, 1), "unit": "steps/s", "n_gpus": 1, "steps": n, "warmup": n_pool,
        "ms_per_step": round(ms_head, 6), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "bf16 weights, f32 accumulation", "data": "synthetic (random weights and hidden states; rotating pool)",
        "config": {"workload": f"indextts-mel-head-{R}x1280x8194", "rows": R, "dim": dim, "vocab": vocab,
                   "pool_weights": n_pool},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None,
                     "algorithmic_bytes_per_launch": step_bytes},
        "fused_head_and_sampler_us": round(ms_fused * 1e3, 3),
    }
    if not args.no_cpu:
        # numpy's f32 matmul (its BLAS threads) and the oracle's sampler on the same rows
        h0, w0, b0 = hidden[0].cpu().numpy(), weights[0].float().cpu().numpy(), bias.cpu().numpy()
        from oracle import oracle as O
        op = O.make_params(O.INDEXTTS, temperature=w.temperature, top_k=w.top_k, top_p=w.top_p, penalty=w.penalty,
                           min_keep=w.min_keep)
        done, t0 = 0, time.perf_counter()
        while time.perf_counter() - t0 < args.cpu_seconds / 2:
            lg = h0 @ w0.T + b0
            O.sample(op, lg, bt.hist_off, bt.hist_ids, bt.uniforms)
            done += 1
        dt = time.perf_counter() - t0
        res["cpu_baseline"] = {"value": round(done / dt, 1), "unit": "steps/s", "cores": host_cpus()[0],
                               "kind": "port", "sample": f"{done} head + sampler steps (numpy f32 matmul, the "
                                                          f"oracle's sampler), {dt:.1f} s"}
    sampler.close()
    print(json.dumps(res), flush=True)


def beam_cpu_baseline(w, bb, nb, seconds: float):
    """The oracle's beam step (C restatement of generation.rs:640-701) on this host."""
    from oracle import oracle as O

    p = O.make_params(w.variant, temperature=w.temperature, top_k=w.top_k, top_p=w.top_p, penalty=w.penalty,
                      min_keep=w.min_keep)
    args = (bb.logits, bb.hist_off, bb.hist_ids, bb.beam_scores, nb, bb.uniforms, 2 * nb)
    O.idx_beam_step(p, *args)
    done, t0 = 0, time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        O.idx_beam_step(p, *args)
        done += 1
    dt = time.perf_counter() - t0
    B = bb.logits.shape[0] // nb
    return {"value": round(done / dt, 2), "unit": "steps/s", "cores": 1, "kind": "port",
            "sample": f"{done} steps of {B} elements x {nb} beams x {w.vocab}, single thread, {dt:.1f} s"}


def main():
    args = parse()
    if args.gpus != 1:
        print("bench.py: this sampler runs on one GPU; multi-GPU runs are not implemented "
              "(rows are independent: each GPU would run the same kernel on its share of the batch)",
              file=sys.stderr)
        sys.exit(2)
    if args.beam:
        return beam_bench(args)
    if args.parity:
        return parity_all(args.parity)
    if args.head:
        return head_bench(args)
    import torch

    from talechime_amd import synth
    from talechime_amd.sampler import DeviceSampler, make_params

    w = synth.WORKLOADS[args.workload]
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    batch = synth.make_batch(w)
    per_batch = w.rows * w.vocab * w.logit_bytes
    n_pool = min(1024, max(2, int(np.ceil(args.pool_mb * 1e6 / per_batch))))
    # pool: the seeded batch first, then batches of the same shape and distribution
    g = torch.Generator(device=dev)
    g.manual_seed(w.seed)
    logits, hists = [], []
    if w.dtype == "bf16":
        first = torch.from_numpy(batch.logits.view(np.int16).copy()).view(torch.bfloat16).to(dev)
    else:
        first = torch.from_numpy(batch.logits).to(dev)
    hoff = torch.from_numpy(batch.hist_off.view(np.int32).copy()).to(dev)
    hid0 = torch.from_numpy((batch.hist_ids if batch.hist_ids.size else np.zeros(1, np.uint32))
                            .view(np.int32).copy()).to(dev)
    for i in range(n_pool):
        if i == 0:
            logits.append(first)
            hists.append(hid0)
        else:
            z = torch.randn(first.shape, generator=g, device=dev, dtype=torch.float32) * w.sigma
            logits.append(z.to(first.dtype))
            hists.append(hid0[torch.randperm(hid0.numel(), generator=g, device=dev)])
    udt = torch.float64 if batch.uniforms.dtype == np.float64 else torch.float32
    unis = [torch.from_numpy(batch.uniforms).to(dev)]
    unis += [torch.rand(batch.uniforms.size, generator=g, device=dev, dtype=udt) for _ in range(n_pool - 1)]
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
    eager_ids = outs[0].ids.clone()
    # host-inclusive rate: K launches from Python (the ctypes call per launch is
    # a few tens of microseconds of host time)
    n_e = min(args.steps, 200)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for i in range(n_e):
        step(i)
    e1.record(stream)
    torch.cuda.synchronize()
    eager_us = e0.elapsed_time(e1) * 1e3 / n_e
    # the timed region: exactly `steps` launches, batch i % n_pool for launch i,
    # captured in HIP graphs (one of the whole pool, one of the remainder) and
    # replayed, so the launches run back to back on the GPU.  The untimed replay
    # of the whole pool before it ends on the last batch, so the first timed
    # batches were last read n_pool - 1 launches (more than the Infinity Cache)
    # earlier.
    K = max(1, args.steps)

    def capture(n):
        if n == 0:
            return None
        side = torch.cuda.Stream(device=dev)
        side.wait_stream(stream)
        with torch.cuda.stream(side):
            for j in range(n):
                step(j)
        stream.wait_stream(side)
        torch.cuda.synchronize()
        gr = torch.cuda.CUDAGraph()
        with torch.cuda.graph(gr):
            for j in range(n):
                step(j)
        return gr

    full = capture(n_pool)
    full_replays, rest = divmod(K, n_pool)
    part = capture(rest)
    full.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(full_replays):
        full.replay()
    if part is not None:
        part.replay()
    e1.record(stream)
    torch.cuda.synchronize()
    steps_done = full_replays * n_pool + rest
    ms_per_step = e0.elapsed_time(e1) / steps_done
    k_avg_us = ms_per_step * 1e3
    # every row of the seeded batch sampled cleanly, and the graph's ids equal the eager launch's
    st = outs[0].status.cpu().numpy()
    if (st != 0).any() or not torch.equal(outs[0].ids, eager_ids):
        print(f"bench.py: {int((st != 0).sum())} rows returned a non-OK status or the graph replay differs",
              file=sys.stderr)
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
    variant = ("qwen", "cosyvoice3", "indextts", "moss", "moss-nano")[w.variant]
    res = {
        "metric": METRIC if w.name == "indextts-mel-256x8194" else f"sampled rows/sec + achieved HBM GB/s ({w.name})",
        "value": round(rows_per_s, 1),
        "unit": "rows/s",
        "n_gpus": 1,
        "steps": steps_done,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32" if w.dtype == "f32" else "bf16",
        "data": f"synthetic (seeded N(0,{w.sigma:g}^2) logits, {w.hist_kind} histories; rotating pool)",
        "config": {"workload": w.name, "rows": w.rows, "vocab": w.vocab, "history": w.hist_len,
                   "penalty": w.penalty, "temperature": w.temperature, "top_k": w.top_k, "top_p": w.top_p,
                   "variant": variant, "pool_batches": n_pool, "seed": w.seed},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": measured_traffic(w.name),
                     "kernel_avg_us": round(k_avg_us, 3), "algorithmic_bytes_per_launch": bytes_per_launch},
        "timing": f"{steps_done} launches: {full_replays} replays of a HIP graph of the {n_pool}-batch pool"
                  + (f" and one of {rest} launches" if rest else "")
                  + f"; launched one by one from Python: {eager_us:.1f} us per step",
    }
    res["parity"] = pool_parity(w, logits, hists, hoff, unis, sampler, params, args.parity_batches)
    if not args.no_cpu:
        res["cpu_baseline"] = cpu_baseline(w, batch, args.cpu_seconds)
    sampler.close()
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
