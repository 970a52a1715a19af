"""Pins of the oracle's typical warper (indextts generation.rs:196-248).

The reference has one vector for it (generation.rs:870-882, in
test_oracle_kats.py).  These tests fix the rest with what the definition
determines, computed here by a different route: the kept set is the
smallest prefix, in ascending order of |surprisal - entropy|, whose softmax
mass reaches `mass`, together with every id tied with the last one; the
entropy, surprisals and masses are taken in float64 from a float64
log-softmax (not the oracle's float32 one), and rows are kept only where the
boundary is far from the float roundings that separate the two.  A wrong
order (descending) or the entropy's sign flipped changes the kept set on
these rows; dropping the ids tied with the cut fails the tie row.  Whether
the running mass is compared with `>=` or `>` cannot be observed: equal
masses would need probabilities exp(s - max) / sum that are exact, which only
ids tied at the maximum (1) or underflowed (0) have.
"""
import numpy as np
import pytest

NEG = -np.inf


def typical_set(scores, mass):
    """Kept ids by the definition, in float64; also the distance of the
    decision from its boundaries (mass and key gaps)."""
    s = np.asarray(scores, np.float64)
    fin = np.isfinite(s)
    m = s[fin].max()
    lse = m + np.log(np.exp(s[fin] - m).sum())
    nz = s - lse
    p = np.where(fin, np.exp(nz), 0.0)
    ent = -(nz[fin] * p[fin]).sum()
    shifted = np.where(fin, np.abs(-nz - ent), np.inf)
    order = np.argsort(shifted, kind="stable")
    cum = np.cumsum(p[order])
    k = int(np.argmax(cum >= mass)) if (cum >= mass).any() else len(order) - 1
    theta = shifted[order[k]]
    keep = shifted <= theta
    # how close the decision is to flipping
    gap_mass = min(abs(cum[k] - mass), abs(cum[k - 1] - mass) if k > 0 else 1.0)
    other = shifted[np.isfinite(shifted) & (shifted != theta)]
    gap_key = np.abs(other - theta).min() if other.size else 1.0
    return keep, gap_mass, gap_key


@pytest.mark.parametrize("seed", range(24))
def test_random_rows_match_the_definition(oracle, seed):
    g = np.random.default_rng(seed)
    V = int(g.integers(3, 60))
    x = (g.standard_normal(V) * g.uniform(0.3, 4.0)).astype(np.float32)
    if seed % 4 == 1:
        x[g.integers(0, V, max(1, V // 5))] = NEG
    mass = float(g.uniform(0.05, 0.98))
    keep, gm, gk = typical_set(x, mass)
    if gm < 1e-6 or gk < 1e-6:
        pytest.skip("the boundary lies within float rounding of the definition")
    out = oracle.idx_typical(x.copy(), mass)
    assert np.array_equal(np.isfinite(out), keep & np.isfinite(x)), (x, mass)
    assert np.array_equal(out[keep], x[keep])


def test_uniform_row_keeps_everything(oracle):
    # every surprisal equals the entropy: one tie group, kept whole
    for V in (2, 7, 64):
        x = np.full(V, 0.25, np.float32)
        out = oracle.idx_typical(x.copy(), 0.3)
        assert np.isfinite(out).all()


def test_ties_at_the_cut_are_kept(oracle):
    # two equal scores straddle the mass: the reference removes only ids
    # strictly beyond the cut's |surprisal - entropy|, so both stay
    x = np.log(np.array([0.4, 0.25, 0.25, 0.1], np.float32)).astype(np.float32)
    keep, _, _ = typical_set(x, 0.5)
    out = oracle.idx_typical(x.copy(), 0.5)
    assert np.array_equal(np.isfinite(out), keep)
    assert np.isfinite(out[1]) and np.isfinite(out[2])


def test_underflowed_ids_go_once_the_mass_is_reached(oracle):
    # ids far below the rest have exactly zero probability and the largest
    # |surprisal - entropy|: any mass below 1 is reached before them
    x = np.array([0.0, 0.0, 0.0, 0.0, -1000.0, -1200.0], np.float32)
    for mass in (0.2, 0.5, 0.99):
        out = oracle.idx_typical(x.copy(), mass)
        assert np.isfinite(out[:4]).all() and (out[4:] == NEG).all()
