"""Shared helpers for the GPU parity tests: run a seeded batch through the HIP
sampler (C ABI) and through the oracle, and compare."""
import numpy as np
import torch

from oracle import oracle as O
from talechime_amd import synth
from talechime_amd.sampler import DeviceSampler, make_params

ORACLE_THREADS = 8


def to_dev(b: synth.Batch, w: synth.Workload, dev="cuda"):
    if w.dtype == "bf16":
        logits = torch.from_numpy(b.logits.view(np.int16).copy()).view(torch.bfloat16).to(dev)
    else:
        logits = torch.from_numpy(b.logits).to(dev)
    ho = torch.from_numpy(b.hist_off.view(np.int32).copy()).to(dev)
    hi = torch.from_numpy((b.hist_ids if b.hist_ids.size else np.zeros(1, np.uint32)).view(np.int32).copy()).to(dev)
    un = torch.from_numpy(b.uniforms).to(dev)
    return logits, ho, hi, un


def params_for(w: synth.Workload, lib: str, **over):
    kw = dict(temperature=w.temperature, top_k=w.top_k, top_p=w.top_p, penalty=w.penalty,
              min_keep=w.min_keep, ras_win=w.ras_win, ras_tau=w.ras_tau)
    kw.update(over)
    if lib == "oracle":
        return O.make_params(w.variant, **kw)
    return make_params(w.variant, **kw)


def run_gpu(sampler: DeviceSampler, w, b, cap=64, **over):
    logits, ho, hi, un = to_dev(b, w)
    p = params_for(w, "gpu", **over)
    r = sampler.sample(p, logits, ho, hi, un, verify_cap=cap)
    torch.cuda.synchronize()
    out = {k: getattr(r, k).cpu().numpy() for k in ("ids", "status", "flags", "topk_count", "topk_ids",
                                                    "keep_count", "keep_ids", "keep_probs", "norm")}
    out["ids"] = out["ids"].view(np.uint32)
    return out


def run_oracle(w, b, cap=64, **over):
    p = params_for(w, "oracle", **over)
    return O.sample(p, b.logits_f32, b.hist_off, b.hist_ids, b.uniforms, cap=cap, nthreads=ORACLE_THREADS)


def set_diff_rows(a, b, cap):
    """Rows whose top-k / keep sets differ (within cap)."""
    bad = []
    for r in range(a["ids"].size):
        for c, i in (("topk_count", "topk_ids"), ("keep_count", "keep_ids")):
            na, nb = int(a[c][r]), int(b[c][r])
            if na != nb:
                bad.append((r, c, na, nb))
                break
            n = min(na, cap)
            if not np.array_equal(a[i][r, :n].astype(np.uint32), b[i][r, :n].astype(np.uint32)):
                bad.append((r, i))
                break
    return bad


def prob_rel_err(a, b, cap):
    worst = 0.0
    for r in range(a["ids"].size):
        n = min(int(a["keep_count"][r]), int(b["keep_count"][r]), cap)
        if n == 0:
            continue
        pa = a["keep_probs"][r, :n].astype(np.float64)
        pb = b["keep_probs"][r, :n].astype(np.float64)
        m = pb > 0
        if m.any():
            worst = max(worst, float(np.max(np.abs(pa[m] - pb[m]) / pb[m])))
    return worst
