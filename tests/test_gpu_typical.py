"""indextts's typical warper (generation.rs:196-248, applied at :649-651) on the
device (k_idx_typical) against the oracle: ids, top-k sets, kept sets and
probabilities, on seeded 8194-logit rows and on small rows with ties, -inf
entries and non-finite scores; both beam steps with the warper on."""
import numpy as np
import pytest

torch = pytest.importorskip("torch")

from oracle import oracle as O  # noqa: E402
from talechime_amd import _lib, synth  # noqa: E402
from talechime_amd.sampler import DeviceSampler, make_params  # noqa: E402
from tests.test_gpu_edges import run, same  # noqa: E402

pytestmark = pytest.mark.gpu
NEAR = 16


@pytest.fixture(scope="module")
def sampler():
    if not torch.cuda.is_available():
        pytest.skip("no GPU visible")
    s = DeviceSampler(0, max_rows=256, max_vocab=16384)
    yield s
    s.close()


def _check(g, o, rows):
    near = (g["flags"] & NEAR) != 0
    print(f"[typical] rows {len(rows)} near {int(near.sum())} statuses {np.unique(g['status'])}", flush=True)
    assert near.sum() == 0
    # rows with more than 1024 survivors: probabilities from block sums
    wide = o["topk_count"] > 1024
    same(g, o, rows=[r for r in rows if not near[r] and not wide[r]])
    same(g, o, rows=[r for r in rows if not near[r] and wide[r]], probs_exact=False)


@pytest.mark.parametrize("mass", [0.9, 0.5, 0.2])
def test_typical_workload_rows(sampler, mass):
    w = synth.WORKLOADS["indextts-mel-256x8194"]
    b = synth.make_batch(w, rows=64, batch_index=3)
    hist = [b.hist_ids[b.hist_off[r]:b.hist_off[r + 1]].tolist() for r in range(64)]
    g, o = run(sampler, O.INDEXTTS, b.logits_f32, hist, b.uniforms, temperature=0.8, top_k=30, top_p=0.8,
               penalty=10.0, min_keep=2, typical=True, typical_mass=mass)
    assert (g["status"] == 0).all(), g["status"]
    _check(g, o, range(64))


@pytest.mark.parametrize("scale", [0.5, 2.0, 6.0])
def test_typical_alone_and_peaked_rows(sampler, scale):
    # no top-k / top-p: the kept set is the typical set itself, also where it
    # exceeds the survivor stage (the register-resident path)
    g_ = np.random.default_rng(int(scale * 10))
    V, rows = 8194, 24
    x = (g_.standard_normal((rows, V)) * scale).astype(np.float32)
    x[:, :3] += np.float32(4 * scale)
    hist = [g_.integers(0, V, 40).tolist() for _ in range(rows)]
    g, o = run(sampler, O.INDEXTTS, x, hist, g_.random(rows), temperature=1.0, top_k=0, top_p=1.0, penalty=1.3,
               min_keep=2, typical=True, typical_mass=0.6)
    if scale < 1.0:
        assert (o["topk_count"] > 1024).all()
    _check(g, o, range(rows))


def test_typical_small_rows_ties_and_infinities(sampler):
    g_ = np.random.default_rng(7)
    V = 300
    rows = []
    for r in range(12):
        x = (g_.standard_normal(V) * 2).astype(np.float32)
        if r % 3 == 1:
            x[g_.integers(0, V, 60)] = -np.inf
        if r % 3 == 2:
            x = np.round(x * 2) / 2  # many ties
        rows.append(x)
    rows.append(np.zeros(V, np.float32))       # one tie group: every id kept
    y = (g_.standard_normal(V)).astype(np.float32)
    y[5] = np.nan                               # NaN score: the reference's mass is NaN, nothing removed
    rows.append(y)
    x = np.stack(rows).astype(np.float32)
    n = x.shape[0]
    hist = [g_.integers(0, V, 10).tolist() for _ in range(n)]
    g, o = run(sampler, O.INDEXTTS, x, hist, g_.random(n), temperature=0.9, top_k=50, top_p=0.95, penalty=1.2,
               min_keep=2, typical=True, typical_mass=0.7)
    _check(g, o, range(n))


def test_typical_in_both_beam_steps(sampler):
    w = synth.WORKLOADS["indextts-mel-256x8194"]
    bb = synth.make_beam_batch(w, 4, 3)
    kw = dict(temperature=0.8, top_k=30, top_p=0.8, penalty=10.0, min_keep=2, typical=True, typical_mass=0.8)
    dev = torch.device("cuda", 0)
    d = {k: torch.from_numpy(np.ascontiguousarray(v)).to(dev) for k, v in
         (("logits", bb.logits), ("ho", bb.hist_off.view(np.int32)), ("hi", bb.hist_ids.view(np.int32)),
          ("bs", bb.beam_scores), ("u", bb.uniforms))}
    c = sampler.beam_step(make_params(_lib.INDEXTTS, **kw), d["logits"], d["ho"], d["hi"], d["bs"], 3, d["u"])
    ob = O.idx_beam_step(O.make_params(O.INDEXTTS, **kw), bb.logits, bb.hist_off, bb.hist_ids, bb.beam_scores,
                         3, bb.uniforms, 6)
    near = (c.flags.cpu().numpy() & NEAR) != 0
    assert near.sum() == 0
    assert np.array_equal(c.flat.cpu().numpy().view(np.uint32), ob["flat"])
    cs = sampler.beam_search_step(make_params(_lib.INDEXTTS, **kw), d["logits"], d["ho"], d["hi"], d["bs"], 3, 6)
    os_ = O.idx_beam_search_step(O.make_params(O.INDEXTTS, **kw), bb.logits, bb.hist_off, bb.hist_ids,
                                 bb.beam_scores, 3, 6)
    assert np.array_equal(cs.flat.cpu().numpy().view(np.uint32), os_["flat"])


def test_typical_mass_is_checked(sampler):
    x = torch.zeros(1, 64, device="cuda")
    u = torch.full((1,), 0.5, dtype=torch.float64, device="cuda")
    for bad in (0.0, 1.0, -0.5, float("nan")):
        with pytest.raises(_lib.TcError):
            sampler.sample(make_params(_lib.INDEXTTS, temperature=0.8, top_k=30, typical=True, typical_mass=bad),
                           x, None, None, u)
