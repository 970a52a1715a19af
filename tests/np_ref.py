"""Independent Python restatement of the five samplers, used to cross-check the
C oracle on random rows.  Written separately from the C code (Python control
flow, numpy float32 scalars for f32 arithmetic, the platform libm through
ctypes for f32 exp/ln so the bits match Rust's f32::exp / f32::ln on Linux).

Slow by design: use on a handful of rows.
"""
import ctypes
import ctypes.util
import math
import struct

import numpy as np

_libm = ctypes.CDLL(ctypes.util.find_library("m"))
_libm.expf.restype = ctypes.c_float
_libm.expf.argtypes = [ctypes.c_float]
_libm.logf.restype = ctypes.c_float
_libm.logf.argtypes = [ctypes.c_float]

F = np.float32
NEG = F(-np.inf)


def expf(x):
    return F(_libm.expf(float(x)))


def logf(x):
    return F(_libm.logf(float(x)))


def total_key(v):
    """Rust f32::total_cmp as an integer key."""
    b = struct.unpack("<I", struct.pack("<f", float(v)))[0]
    return (~b) & 0xFFFFFFFF if b & 0x80000000 else b | 0x80000000


def fsum_seq(vals, start=F(-0.0)):
    s = F(start)
    for v in vals:
        s = F(s + F(v))
    return s


# ------------------------------------------------------------------ qwen
def qwen_row(x, *, temperature, top_k, top_p, penalty, seen_ids, u, add_mask=None, eos_id=-1):
    x = [F(v) for v in x]
    V = len(x)
    if abs(penalty - 1.0) >= 1e-9:
        pf = F(penalty)
        inv = F(F(1.0) / pf)
        mask = set(int(i) for i in seen_ids if int(i) < V)
        for i in mask:
            x[i] = F(x[i] * (inv if x[i] > 0 else pf))
    if add_mask is not None:
        x = [F(a + F(b)) for a, b in zip(x, add_mask)]
    if 0 <= eos_id < V:
        x[eos_id] = NEG
    if temperature != 1.0 and temperature > 0.0:
        m = F(1.0 / temperature)
        x = [F(F(v * m) + F(0.0)) for v in x]
    if temperature < 0.01:
        best, acc = 0, x[0]
        for i, v in enumerate(x):
            if acc < v:
                acc, best = v, i
        return best
    if top_k > 0:
        k = min(top_k, V)
        thr = sorted(x, key=lambda v: -float(v))[k - 1]
        x = [v if v >= thr else NEG for v in x]
    if 0.0 < top_p < 1.0:
        order = sorted(range(V), key=lambda i: (-float(x[i]), i))
        mx = x[order[0]]
        e = [expf(F(x[i] - mx)) for i in order]
        s = fsum_seq(e)
        cum, cut = F(0.0), V
        for j, ev in enumerate(e):
            cum = F(cum + F(ev / s))
            if cum > F(top_p):
                cut = j + 1
                break
        keep = set(order[:cut])
        x = [v if i in keep else NEG for i, v in enumerate(x)]
    mx = x[0]
    for v in x[1:]:
        mx = v if np.isnan(mx) else (mx if np.isnan(v) else max(mx, v))
    e = [expf(F(v - mx)) for v in x]
    s = fsum_seq(e, F(0.0))
    cum = F(0.0)
    for i, ev in enumerate(e):
        cum = F(cum + F(ev / s))
        if cum >= F(u):
            return i
    return 0


# ------------------------------------------------------------------ cosyvoice3
def cosy_row(x, *, top_p, top_k, win, tau, hist, u0, u1, eos_id=-1):
    x = [F(v) for v in x]
    V = len(x)
    if eos_id >= 0:
        x = [F(v + (NEG if i == eos_id else F(0.0))) for i, v in enumerate(x)]
    mx = x[0]
    for v in x[1:]:
        mx = max(mx, v)
    e = [expf(F(v - mx)) for v in x]
    s = fsum_seq(e, F(0.0))
    p = [F(ev / s) for ev in e]
    order = sorted(range(V), key=lambda i: (-total_key(p[i]), i))
    if 0 < top_k < V:
        order = order[: top_k + 1]
    cum, cands = F(0.0), []
    for i in order:
        if cum < F(top_p) and len(cands) < top_k:
            cum = F(cum + p[i])
            cands.append(i)
        else:
            break
    if not cands:
        top = order[0]
    else:
        total = fsum_seq([p[i] for i in cands])
        pick = F(F(u0) * total)
        acc, top = F(0.0), cands[-1]
        for i in cands:
            acc = F(acc + p[i])
            if pick < acc:
                top = i
                break
    recent = list(hist)[-win:] if win else []
    rep = sum(1 for t in recent if t == top)
    if F(rep) >= F(F(win) * F(tau)):
        acc = F(0.0)
        for i in range(V):
            acc = F(acc + p[i])
            if F(u1) < acc:
                return i, True
        return V - 1, True
    return top, False


# ------------------------------------------------------------------ indextts
def indextts_scores(x, *, temperature, top_k, top_p, penalty, hist, min_keep=2):
    """The processors of one row (generation.rs:643-662); f32 scores."""
    s = [F(v) for v in x]
    V = len(s)
    mx = F(-np.inf)
    for v in s:
        mx = v if v > mx else mx
    if np.isfinite(mx):
        tot = fsum_seq([expf(F(v - mx)) for v in s])
        L = logf(tot)
        s = [F(F(v - mx) - L) for v in s]
    if penalty != 1.0:
        orig = list(s)
        pf = F(penalty)
        for i in hist:
            i = int(i)
            if i < V:
                o = orig[i]
                s[i] = F(o * pf) if o < 0 else F(o / pf)
    if temperature != 1.0:
        t = F(temperature)
        s = [F(v / t) for v in s]
    if top_k != 0:
        k = min(max(top_k, min_keep), V)
        if 0 < k < V:
            kth = sorted(s, key=lambda v: -total_key(v))[k - 1]
            s = [NEG if v < kth else v for v in s]
    if top_p < 1.0:
        d = [float(v) for v in s]
        m = max(d)
        ex = [math.exp(v - m) for v in d]
        tot = -0.0
        for v in ex:
            tot += v
        probs = [v / tot for v in ex]
        order = [i for i in range(V) if s[i] != NEG]
        order.sort(key=lambda i: (total_key(s[i]), i))
        remove = set()
        cum = 0.0
        for i in order:
            cum += probs[i]
            if cum <= 1.0 - top_p:
                remove.add(i)
        for i in order[::-1][:min_keep]:
            remove.discard(i)
        s = [NEG if i in remove else v for i, v in enumerate(s)]
    return s


def wo_replacement(joint, n, us):
    """sample_without_replacement (generation.rs:280-303) over f64 scores with
    the uniforms us[0..n); None when fewer than n are finite."""
    live = [i for i in range(len(joint)) if math.isfinite(joint[i])]
    if len(live) < n:
        return None
    out = []
    for d in range(n):
        m = max(joint[i] for i in live)
        ex = [math.exp(joint[i] - m) for i in live]
        tot = -0.0
        for v in ex:
            tot += v
        w = [v / tot for v in ex]
        total = -0.0
        for v in w:
            total += v
        uu = us[d] * total
        acc, last, pick = 0.0, 0, None
        for j, wv in enumerate(w):
            if wv <= 0.0:
                continue
            last = j
            acc += wv
            if acc > uu:
                pick = j
                break
        pick = last if pick is None else pick
        out.append(live.pop(pick))
    return out


def indextts_row(x, *, temperature, top_k, top_p, penalty, hist, u, min_keep=2):
    s = indextts_scores(x, temperature=temperature, top_k=top_k, top_p=top_p, penalty=penalty, hist=hist,
                        min_keep=min_keep)
    r = wo_replacement([float(v) + 0.0 for v in s], 1, [u])
    return None if r is None else r[0]


def indextts_beam_step(rows, hists, bonus, num_beams, us, n_draws, **kw):
    """generation.rs:640-701 for one batch element: the beam rows' scores
    joined beam-major with each row's running score added, n_draws draws,
    candidates (score, flat) sorted by score descending (a stable sort)."""
    joint = []
    for j in range(num_beams):
        s = indextts_scores(rows[j], hist=hists[j], **kw)
        joint += [float(v) + float(bonus[j]) for v in s]
    picks = wo_replacement(joint, n_draws, us)
    if picks is None:
        return None
    return sorted([(joint[f], f) for f in picks], key=lambda c: -c[0])


# ------------------------------------------------------------------ moss
def moss_row(x, *, temperature, top_k, top_p, penalty, hist, u, exclude=-1):
    v = [F(a) for a in x]
    pen, T = F(penalty), F(temperature)
    for i in set(int(h) for h in hist):
        if i < len(v):
            v[i] = F(v[i] * pen) if v[i] < 0 else F(v[i] / pen)
    if exclude >= 0:
        v[exclude] = NEG
    ranked = sorted(range(len(v)), key=lambda i: (-total_key(v[i]), i))
    if T == 0:
        return ranked[0]
    ranked = ranked[: min(top_k, len(v))]
    mx = v[ranked[0]]
    w = [float(expf(F(F(v[i] - mx) / T))) for i in ranked]
    total = -0.0
    for a in w:
        total += a
    cum, keep = 0.0, len(w)
    for j, a in enumerate(w):
        cum += a / total
        if cum > top_p:
            keep = j + 1
            break
    w = w[:keep]
    sw = -0.0
    for a in w:
        sw += a
    draw = u * sw
    for j, a in enumerate(w):
        draw -= a
        if draw <= 0.0:
            return ranked[j]
    return ranked[keep - 1]


def nano_row(x, *, temperature, top_k, top_p, penalty, hist, u):
    s = [F(a) for a in x]
    pen, T = F(penalty), F(temperature)
    for i in set(int(h) for h in hist):
        s[i] = F(s[i] * pen) if s[i] < 0 else F(s[i] / pen)
    s = [F(a / T) for a in s]
    ranked = sorted(range(len(s)), key=lambda i: (-total_key(s[i]), i))
    thr = s[ranked[min(top_k, len(s)) - 1]]
    mx = s[ranked[0]]
    w = [0.0 if a < thr else math.exp(float(F(a - mx))) for a in s]
    if top_p < 1.0:
        total = -0.0
        for a in w:
            total += a
        cum = 0.0
        for i in ranked:
            if cum > top_p:
                w[i] = 0.0
            else:
                cum += w[i] / total
    sw = -0.0
    for a in w:
        sw += a
    draw = u * sw
    for i, a in enumerate(w):
        draw -= a
        if a > 0.0 and draw <= 0.0:
            return i
    return None
