"""Pins of the oracle's moss sampler (moss-tts/src/sampling.rs:22-85).

The reference has no vectors for the moss draw beyond its errors and greedy
path, so these tests fix it with what the mathematics determines:

- rows of equal finite logits (every weight exactly 1.0, cumulative shares
  exact multiples of 1/n), which separate `cumulative > top_p` from `>=`,
  truncation at `keep` from truncation at `top_k`, and the `ranked[keep-1]`
  fallback from the other candidates;
- the rank (value-descending) order of the CDF on rows whose vocabulary order
  differs from it;
- a brute force over a grid of uniforms on small rows, against the exact
  inverse-CDF interval of each rank computed independently in double;
- the probabilities against exp((v - max)/T) evaluated in double, and the
  penalty's dedupe and sign rule by the same route.

Ties among equal logits are ordered by ascending id in the oracle (Rust's
sort_unstable_by leaves them unspecified) and the row is flagged TIE_CUT
when the order decides a cut.
"""
import math

import numpy as np
import pytest

TIE_CUT = 1


def moss(oracle, x, u, *, T=1.0, k=None, p=1.0, pen=1.0, hist=(), exclude=-1, cap=64):
    x = np.asarray([x], np.float32)
    V = x.shape[1]
    k = V if k is None else k
    h = np.asarray(hist, np.uint32)
    prm = oracle.make_params(oracle.MOSS, temperature=T, top_k=k, top_p=p, penalty=pen, exclude_id=exclude)
    r = oracle.sample(prm, x, np.array([0, h.size], np.uint32), h, np.array([u], np.float64), cap=cap)
    return r


def kept(r):
    return [int(i) for i in r["keep_ids"][0][: int(r["keep_count"][0])]]


# ------------------------------------------------ exact-share rows (weights 1.0)
@pytest.mark.parametrize("p,keep", [(0.0, 1), (0.125, 2), (0.375, 4), (0.5, 5), (0.875, 8),
                                    (0.999, 8), (1.0, 8)])
def test_top_p_crossing_is_strict_and_kept(oracle, p, keep):
    # 8 equal logits: cumulative after rank i is (i+1)/8 exactly.  keep is the
    # first i+1 with cumulative > p (strict: at p = 0.5 rank 3 reaches 0.5 and
    # does not stop the loop; rank 4 does and is kept).  Never exceeding
    # (p = 1.0) keeps all.
    r = moss(oracle, [0.0] * 8, 0.0, p=p)
    assert r["status"][0] == 0
    assert int(r["keep_count"][0]) == keep
    assert kept(r) == list(range(keep))  # ties ranked by ascending id
    assert bool(r["flags"][0] & TIE_CUT) == (keep < 8)


@pytest.mark.parametrize("u", [0.0, 1 / 16, 0.25, 0.5, 0.625, 15 / 16, 1.0])
def test_draw_subtracts_in_rank_order(oracle, u):
    # keep = 4 of 8 equal weights (p = 0.375): draw = u * 4 exactly; draw -= 1
    # per rank and the first draw <= 0 picks, so rank max(ceil(4u) - 1, 0).
    r = moss(oracle, [0.0] * 8, u, p=0.375)
    want = max(math.ceil(4 * u) - 1, 0)
    assert int(r["ids"][0]) == want


def test_fallback_is_last_kept_rank(oracle):
    # a uniform above 1 leaves draw > 0 after every kept weight: the reference
    # returns ranked[keep - 1], not ranked[0] and not ranked[top_k - 1]
    r = moss(oracle, [0.0] * 8, 1.5, p=0.375)
    assert int(r["keep_count"][0]) == 4 and int(r["ids"][0]) == 3
    r = moss(oracle, [0.0] * 8, 1.5, k=6, p=1.0)
    assert int(r["ids"][0]) == 5


def test_draw_is_truncated_at_keep(oracle):
    # u = 0.999 scales the kept sum (4), not the top-k sum (8): rank 3, not 7
    r = moss(oracle, [0.0] * 8, 0.999, p=0.375)
    assert int(r["ids"][0]) == 3
    # top_k truncates before top-p: k = 3 of 8 equal weights, shares 1/3
    r = moss(oracle, [0.0] * 8, 0.999, k=3, p=1.0)
    assert int(r["topk_count"][0]) == 3 and int(r["ids"][0]) == 2
    assert r["flags"][0] & TIE_CUT


def test_minus_inf_entries_rank_last_with_zero_weight(oracle):
    # -inf logits sort after every finite one and weigh exactly 0
    x = [-np.inf, 0.0, -np.inf, 0.0, 0.0, -np.inf, 0.0, -np.inf]
    r = moss(oracle, x, 0.999, k=8, p=1.0)
    assert int(r["ids"][0]) == 6
    # every rank is kept (the share never exceeds 1); verification lists ids ascending
    probs = dict(zip(kept(r), r["keep_probs"][0].tolist()))
    assert probs == {0: 0.0, 1: 0.25, 2: 0.0, 3: 0.25, 4: 0.25, 5: 0.0, 6: 0.25, 7: 0.0}
    for u in (0.0, 0.3, 0.6, 1.0):
        assert np.isfinite(x[int(moss(oracle, x, u, k=8, p=1.0)["ids"][0])])


# ------------------------------------------------ rank order and brute force
def test_cdf_runs_in_rank_order(oracle):
    # vocabulary order 0..3, rank order 1, 3, 2, 0
    x = [0.0, 3.0, 1.0, 2.0]
    assert int(moss(oracle, x, 0.01)["ids"][0]) == 1
    assert int(moss(oracle, x, 0.999)["ids"][0]) == 0


def _exact_token(x, u, T, k, p):
    """Independent evaluation in double: rank order, top-k, strict top-p share,
    inverse CDF over the kept weights.  Returns None within 1e-6 of a decision."""
    order = sorted(range(len(x)), key=lambda i: (-x[i], i))[:k]
    m = x[order[0]]
    w = [math.exp((x[i] - m) / T) for i in order]
    tot = math.fsum(w)
    cum, keep = 0.0, len(w)
    for i, wi in enumerate(w[:-1]):  # a crossing at the last rank keeps them all anyway
        cum += wi / tot
        if abs(cum - p) < 1e-6:
            return None
        if cum > p:
            keep = i + 1
            break
    s = math.fsum(w[:keep])
    d, acc = u * s, 0.0
    for i in range(keep):
        acc += w[i]
        if abs(acc - d) < 1e-6 * s:
            return None
        if d <= acc:
            return order[i]
    return order[keep - 1]


@pytest.mark.parametrize("seed", range(6))
def test_brute_force_uniform_grid_small_rows(oracle, seed):
    g = np.random.default_rng(100 + seed)
    V = int(g.integers(2, 9))
    x = (g.standard_normal(V) * 2).astype(np.float32)
    T = float(np.float32(g.choice([0.5, 0.8, 1.0, 1.7])))
    k = int(g.integers(1, V + 1))
    p = float(g.choice([0.3, 0.6, 0.8, 1.0]))
    xs = [float(v) for v in x]
    checked = 0
    for j in range(257):
        u = j / 256
        want = _exact_token(xs, u, T, k, p)
        if want is None:
            continue
        got = int(moss(oracle, x, u, T=T, k=k, p=p, cap=0)["ids"][0])
        assert got == want, (seed, u, got, want)
        checked += 1
    assert checked > 200


def test_probabilities_temperature_inside_exp(oracle):
    # keep_probs = w / sum(kept w), w = exp((v - max) / T) in f32 then widened
    x = [0.5, -1.25, 2.0, 1.0, -3.0]
    T = 0.7
    r = moss(oracle, x, 0.3, T=T, p=1.0)
    order = sorted(range(5), key=lambda i: -x[i])
    w = {i: math.exp((x[i] - x[order[0]]) / np.float32(T)) for i in order}
    s = math.fsum(w.values())
    for i, pr in zip(kept(r), r["keep_probs"][0]):
        assert abs(pr - w[i] / s) <= 1e-6 * (w[i] / s)


def test_penalty_dedupe_and_sign(oracle):
    # values[id] < 0 -> * penalty, else / penalty, once per distinct id
    x = [2.0, -2.0, 1.5]
    r = moss(oracle, x, 0.3, pen=2.0, hist=[0, 0, 1, 1, 1])
    v = [1.0, -4.0, 1.5]
    w = [math.exp(t - 1.5) for t in v]
    s = math.fsum(w)
    got = dict(zip(kept(r), r["keep_probs"][0]))
    for i in range(3):
        assert abs(got[i] - w[i] / s) <= 1e-6 * (w[i] / s)


def test_exclude_and_greedy(oracle):
    x = [0.0, 5.0, 1.0, 4.0]
    # the excluded id ranks last with weight exactly 0: kept by the share loop,
    # never drawn
    for u in (0.0, 0.5, 0.999, 1.0):
        r = moss(oracle, x, u, exclude=1)
        assert int(r["ids"][0]) != 1
    assert dict(zip(kept(r), r["keep_probs"][0].tolist()))[1] == 0.0
    r = moss(oracle, x, 0.5, T=0.0, exclude=1)
    assert int(r["ids"][0]) == 3
