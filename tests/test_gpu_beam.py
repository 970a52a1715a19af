"""Parity of the indextts beam-sample step (tc_indextts_beam_step, through the
C ABI) with the oracle's restatement of generation.rs:640-701.

Bar: candidate flat indices and joint scores bit-exact per batch element.
Elements carrying TC_FLAG_NEAR_TIE (a top-p or draw decision within the f64
exp error of the reference's libm) are counted, and only they may differ.
"""
import numpy as np
import pytest

torch = pytest.importorskip("torch")

from oracle import oracle as O  # noqa: E402
from talechime_amd import _lib, synth  # noqa: E402

pytestmark = pytest.mark.gpu

W = synth.WORKLOADS["indextts-mel-256x8194"]


@pytest.fixture(scope="module")
def sampler():
    if not torch.cuda.is_available():
        pytest.skip("no GPU visible")
    from talechime_amd.sampler import DeviceSampler
    s = DeviceSampler(0, max_rows=1024, max_vocab=1 << 14)
    yield s
    s.close()


def _kw(**over):
    kw = dict(temperature=W.temperature, top_k=W.top_k, top_p=W.top_p, penalty=W.penalty, min_keep=2)
    kw.update(over)
    return kw


def _run(sampler, logits, hist_off, hist_ids, bonus, nb, uniforms, n_draws, **kw):
    from talechime_amd.sampler import make_params
    x = np.ascontiguousarray(logits, np.float32)
    dho = dhi = None
    if hist_off is not None:
        dho = torch.from_numpy(np.asarray(hist_off, np.uint32).view(np.int32).copy()).cuda()
        ids = np.asarray(hist_ids, np.uint32)
        dhi = torch.from_numpy((ids if ids.size else np.zeros(1, np.uint32)).view(np.int32).copy()).cuda()
    p = make_params(_lib.INDEXTTS, penalty=kw.pop("penalty", 1.0), **kw)
    r = sampler.beam_step(p, torch.from_numpy(x).cuda(), dho, dhi, torch.from_numpy(np.asarray(bonus, np.float64)).cuda(),
                          nb, torch.from_numpy(np.asarray(uniforms, np.float64)).cuda(), n_draws)
    torch.cuda.synchronize()
    return {"flat": r.flat.cpu().numpy().view(np.uint32), "scores": r.scores.cpu().numpy(),
            "status": r.status.cpu().numpy(), "flags": r.flags.cpu().numpy()}


def _compare(g, o, name, **info):
    near = (g["flags"] & 16) != 0
    ok = ~near
    assert np.array_equal(g["status"], o["status"]), (g["status"], o["status"])
    good = ok & (o["status"] == 0)
    diff = [bi for bi in np.nonzero(good)[0]
            if not (np.array_equal(g["flat"][bi], o["flat"][bi])
                    and np.array_equal(g["scores"][bi].view(np.int64), o["scores"][bi].view(np.int64)))]
    print(f"[beam] {name} " + " ".join(f"{k}={v}" for k, v in info.items())
          + f" elements={g['status'].size} near_tie={int(near.sum())} mismatch={len(diff)}", flush=True)
    assert not diff, [(bi, g["flat"][bi], o["flat"][bi]) for bi in diff[:3]]


@pytest.mark.parametrize("first_step", [True, False])
@pytest.mark.parametrize("batch_index", [0, 1])
def test_beam_step_workload(sampler, first_step, batch_index):
    # 64 elements x 3 beams of the indextts mel-code rows (8194 f32 logits,
    # history 1500, penalty 10, T 0.8, top-k 30, top-p 0.8), six draws each
    bb = synth.make_beam_batch(W, 64, 3, first_step=first_step, batch_index=batch_index)
    args = (bb.logits, bb.hist_off, bb.hist_ids, bb.beam_scores, 3, bb.uniforms, 6)
    g = _run(sampler, *args, **_kw())
    o = O.idx_beam_step(O.make_params(O.INDEXTTS, **_kw()), *args)
    assert (o["status"] == 0).all()
    _compare(g, o, "workload", first_step=first_step, batch=batch_index)
    if first_step:
        # the active beam's kept ids are drawn before the inactive beams refill
        assert (g["flat"][:, :2] < W.vocab).all()


@pytest.mark.parametrize("top_k,nb,top_p", [(200, 2, 0.8), (0, 1, 1.0), (5, 4, 0.8), (40, 3, 1.0), (100, 2, 1.0)])
def test_beam_step_shapes(sampler, top_k, nb, top_p):
    # top-k 200: the general row path; top-k 0 with top-p 1: every finite score
    # of a small vocabulary is live (700 joint entries, staged in LDS); 4 beams
    # of top-k 5; 120 and 200 joint entries (two and four per lane)
    g_ = np.random.default_rng(top_k + nb)
    V = 8194 if top_k else 700
    batch = 6
    x = (g_.standard_normal((batch * nb, V)) * 4).astype(np.float32)
    hist = g_.integers(0, V, (batch * nb, 40)).astype(np.uint32)
    off = (np.arange(batch * nb + 1) * 40).astype(np.uint32)
    bonus = -g_.random(batch * nb) * 10
    n_draws = 2 * nb
    u = g_.random(batch * n_draws)
    kw = _kw(top_k=top_k, top_p=top_p)
    g = _run(sampler, x, off, hist.reshape(-1), bonus, nb, u, n_draws, **kw)
    o = O.idx_beam_step(O.make_params(O.INDEXTTS, **kw), x, off, hist.reshape(-1), bonus, nb, u, n_draws)
    _compare(g, o, "shapes", top_k=top_k, nb=nb)


def test_beam_step_too_few_and_nan_rows(sampler):
    g_ = np.random.default_rng(9)
    V, nb = 300, 3
    x = (g_.standard_normal((4 * nb, V)) * 3).astype(np.float32)
    x[1, 7] = np.nan  # beam 1 of element 0: every score NaN, nothing live in it
    kw = _kw(top_k=2, top_p=0.1, penalty=1.0)
    bonus = np.zeros(4 * nb)
    # two kept ids per live row: element 0 has 4 finite joint scores, the others 6
    for n_draws, want_ok in ((4, [1, 1, 1, 1]), (6, [0, 1, 1, 1]), (7, [0, 0, 0, 0])):
        u = g_.random(4 * n_draws)
        g = _run(sampler, x, None, None, bonus, nb, u, n_draws, **kw)
        o = O.idx_beam_step(O.make_params(O.INDEXTTS, **kw), x, None, None, bonus, nb, u, n_draws)
        assert list(o["status"] == 0) == [bool(v) for v in want_ok]
        _compare(g, o, "too-few", n_draws=n_draws)


def test_beam_step_rejects_bad_arguments(sampler):
    from talechime_amd.sampler import make_params
    x = torch.zeros(6, 100, device="cuda")
    b = torch.zeros(6, dtype=torch.float64, device="cuda")
    u = torch.zeros(12, dtype=torch.float64, device="cuda")
    with pytest.raises(ValueError):
        sampler.beam_step(make_params(_lib.QWEN), x, None, None, b, 3, u)
    p = make_params(_lib.INDEXTTS, top_k=5)
    with pytest.raises(_lib.TcError):  # more than 64 draws
        sampler.beam_step(p, x, None, None, b, 3, torch.zeros(2 * 65, dtype=torch.float64, device="cuda"), 65)
    L = _lib.load()
    cf = torch.zeros(12, dtype=torch.int32, device="cuda")
    cs = torch.zeros(12, dtype=torch.float64, device="cuda")
    st = torch.zeros(2, dtype=torch.int32, device="cuda")
    s = torch.cuda.current_stream().cuda_stream
    import ctypes
    rc = L.tc_indextts_beam_step(sampler.ctx, ctypes.byref(p), x.data_ptr(), 0, 2, 0, 100, 100, None, None,
                                 b.data_ptr(), u.data_ptr(), 6, cf.data_ptr(), cs.data_ptr(), st.data_ptr(), None, s)
    assert rc == _lib.TC_EINVAL  # num_beams 0


def test_beam_step_concentrated_refill(sampler):
    # generation.rs:917-935 on logits: each beam row keeps two ids (top-k 2),
    # the first step's beam scores are 0, -1e9, -1e9.  The active beam's two ids
    # are drawn first; the inactive beams' ids (weights exactly 0 until then)
    # refill the other four draws.
    g_ = np.random.default_rng(21)
    V, nb, batch = 500, 3, 8
    x = (g_.standard_normal((batch * nb, V)) * 3).astype(np.float32)
    bonus = np.array([0.0 if r % nb == 0 else -1e9 for r in range(batch * nb)])
    u = g_.random(batch * 6)
    kw = _kw(top_k=2, top_p=1.0, penalty=1.0)
    g = _run(sampler, x, None, None, bonus, nb, u, 6, **kw)
    o = O.idx_beam_step(O.make_params(O.INDEXTTS, **kw), x, None, None, bonus, nb, u, 6)
    assert (o["status"] == 0).all()
    _compare(g, o, "refill")
    assert (g["flat"][:, :2] < V).all() and all(len(set(r)) == 6 for r in g["flat"].tolist())


def test_beam_step_boundary_draws_take_the_exact_path(sampler):
    # four equal kept scores: weights 0.25 and a uniform of 0.5 put the target
    # on a running sum exactly (acc > u fails at the second entry).  The draw
    # falls inside the margin, runs the reference's sequential loops and is
    # flagged; exp(0) = 1 is exact, so the candidates still equal the oracle's.
    V, nb, batch = 64, 1, 4
    x = np.full((batch, V), -30.0, np.float32)
    x[:, [3, 17, 40, 41]] = 2.0
    u = np.tile([0.5, 0.5, 0.25, 0.999], batch)
    kw = _kw(top_k=4, top_p=1.0, penalty=1.0)
    g = _run(sampler, x, None, None, np.zeros(batch), nb, u, 4, **kw)
    o = O.idx_beam_step(O.make_params(O.INDEXTTS, **kw), x, None, None, np.zeros(batch), nb, u, 4)
    assert (g["flags"] & 16).all()
    assert np.array_equal(g["flat"], o["flat"]) and np.array_equal(g["scores"], o["scores"])


def test_beam_step_bf16_rows(sampler):
    # bf16 logits are widened exactly (to_dtype(F32)); the oracle sees the same values
    from talechime_amd.synth import bf16_bits_to_f32, to_bf16_bits
    from talechime_amd.sampler import make_params
    g_ = np.random.default_rng(5)
    V, nb, batch = 8194, 3, 8
    x = (g_.standard_normal((batch * nb, V)) * 4).astype(np.float32)
    bits = to_bf16_bits(x)
    xf = bf16_bits_to_f32(bits)
    bonus = -g_.random(batch * nb) * 20
    u = g_.random(batch * 6)
    p = make_params(_lib.INDEXTTS, **_kw(penalty=1.0))
    r = sampler.beam_step(p, torch.from_numpy(bits.view(np.int16)).view(torch.bfloat16).cuda(), None, None,
                          torch.from_numpy(bonus).cuda(), nb, torch.from_numpy(u).cuda())
    torch.cuda.synchronize()
    g = {"flat": r.flat.cpu().numpy().view(np.uint32), "scores": r.scores.cpu().numpy(),
         "status": r.status.cpu().numpy(), "flags": r.flags.cpu().numpy()}
    o = O.idx_beam_step(O.make_params(O.INDEXTTS, **_kw(penalty=1.0)), xf, None, None, bonus, nb, u, 6)
    _compare(g, o, "bf16")


@pytest.mark.parametrize("first_step", [True, False])
@pytest.mark.parametrize("batch_index", [0, 1])
def test_beam_search_step_matches_oracle(sampler, first_step, batch_index):
    # do_sample = false (generation.rs:671-679): the 6 best joint scores of
    # each of 64 elements x 3 beams, bit for bit; the sampling warpers set in
    # the parameters are not applied
    from talechime_amd.sampler import make_params
    bb = synth.make_beam_batch(W, 64, 3, first_step=first_step, batch_index=batch_index)
    dho = torch.from_numpy(bb.hist_off.view(np.int32).copy()).cuda()
    dhi = torch.from_numpy(bb.hist_ids.view(np.int32).copy()).cuda()
    p = make_params(_lib.INDEXTTS, **_kw())
    r = sampler.beam_search_step(p, torch.from_numpy(bb.logits).cuda(), dho, dhi,
                                 torch.from_numpy(bb.beam_scores).cuda(), 3)
    torch.cuda.synchronize()
    o = O.idx_beam_search_step(O.make_params(O.INDEXTTS, **_kw()), bb.logits, bb.hist_off, bb.hist_ids,
                               bb.beam_scores, 3, 6)
    assert (r.status.cpu().numpy() == 0).all()
    assert np.array_equal(r.flat.cpu().numpy().view(np.uint32), o["flat"])
    assert np.array_equal(r.scores.cpu().numpy().view(np.int64), o["scores"].view(np.int64))


def test_beam_search_step_ties_in_flat_order(sampler):
    # two beams with equal rows, histories and beam scores: every joint score
    # is tied across them and beam 0's flat index comes first
    from talechime_amd.sampler import make_params
    g = np.random.default_rng(3)
    V = W.vocab
    x = (g.standard_normal((3, V)) * 4).astype(np.float32)
    x[1] = x[0]
    hist = [g.integers(0, V, 200).astype(np.uint32)] * 2 + [g.integers(0, V, 200).astype(np.uint32)]
    off = np.zeros(4, np.uint32)
    off[1:] = np.cumsum([h.size for h in hist])
    ids = np.concatenate(hist)
    bonus = np.array([-1.5, -1.5, -40.0])
    p = make_params(_lib.INDEXTTS, **_kw())
    r = sampler.beam_search_step(p, torch.from_numpy(x).cuda(), torch.from_numpy(off.view(np.int32)).cuda(),
                                 torch.from_numpy(ids.view(np.int32)).cuda(), torch.from_numpy(bonus).cuda(), 3)
    torch.cuda.synchronize()
    o = O.idx_beam_search_step(O.make_params(O.INDEXTTS, **_kw()), x, off, ids, bonus, 3, 6)
    f = r.flat.cpu().numpy().view(np.uint32)[0]
    assert np.array_equal(f, o["flat"][0])
    assert [int(v) // V for v in f] == [0, 1] * 3
