"""Cross-check the C oracle against the independent Python restatement
(tests/np_ref.py) on seeded rows of every workload and on small random rows.
"""
import numpy as np
import pytest

from talechime_amd import synth
from tests import np_ref


def _rows(w, n):
    b = synth.make_batch(w, rows=n)
    return b


@pytest.mark.parametrize("name", ["qwen-talker-1x3072", "qwen-cp-512x2048"])
def test_qwen_rows(oracle, name):
    w = synth.WORKLOADS[name]
    b = _rows(w, min(w.rows, 4))
    p = oracle.make_params(oracle.QWEN, temperature=w.temperature, top_k=w.top_k, top_p=w.top_p,
                           penalty=w.penalty)
    r = oracle.sample(p, b.logits_f32, b.hist_off, b.hist_ids, b.uniforms)
    for i in range(b.logits_f32.shape[0]):
        h = b.hist_ids[b.hist_off[i]:b.hist_off[i + 1]]
        want = np_ref.qwen_row(b.logits_f32[i], temperature=w.temperature, top_k=w.top_k,
                               top_p=w.top_p, penalty=w.penalty, seen_ids=h, u=b.uniforms[i])
        assert r["ids"][i] == want


def test_cosy_rows(oracle):
    w = synth.WORKLOADS["cosy-ras-128x6564"]
    b = _rows(w, 40)  # includes spiked rows 7 and 39
    p = oracle.make_params(oracle.COSY_RAS, top_k=w.top_k, top_p=w.top_p, ras_win=w.ras_win,
                           ras_tau=w.ras_tau)
    r = oracle.sample(p, b.logits_f32, b.hist_off, b.hist_ids, b.uniforms)
    fired = 0
    for i in (0, 1, 7, 39):
        h = b.hist_ids[b.hist_off[i]:b.hist_off[i + 1]]
        want, ras = np_ref.cosy_row(b.logits_f32[i], top_p=w.top_p, top_k=w.top_k, win=w.ras_win,
                                    tau=w.ras_tau, hist=h, u0=b.uniforms[2 * i],
                                    u1=b.uniforms[2 * i + 1])
        assert r["ids"][i] == want
        assert bool(r["flags"][i] & oracle.FLAG_RAS) == ras
        fired += ras
    assert fired >= 1  # row 7 repeats its spiked id inside the window


def test_indextts_rows(oracle):
    w = synth.WORKLOADS["indextts-mel-256x8194"]
    b = _rows(w, 3)
    p = oracle.make_params(oracle.INDEXTTS, temperature=w.temperature, top_k=w.top_k, top_p=w.top_p,
                           penalty=w.penalty, min_keep=2)
    r = oracle.sample(p, b.logits_f32, b.hist_off, b.hist_ids, b.uniforms)
    for i in range(3):
        h = b.hist_ids[b.hist_off[i]:b.hist_off[i + 1]]
        want = np_ref.indextts_row(b.logits_f32[i], temperature=w.temperature, top_k=w.top_k,
                                   top_p=w.top_p, penalty=w.penalty, hist=h, u=b.uniforms[i])
        assert r["ids"][i] == want


def test_qwen_stress_row(oracle):
    w = synth.WORKLOADS["qwen-stress-256x151936"]
    b = _rows(w, 1)
    p = oracle.make_params(oracle.QWEN, temperature=w.temperature, top_k=w.top_k, top_p=w.top_p,
                           penalty=w.penalty)
    r = oracle.sample(p, b.logits_f32, b.hist_off, b.hist_ids, b.uniforms)
    h = b.hist_ids[b.hist_off[0]:b.hist_off[1]]
    want = np_ref.qwen_row(b.logits_f32[0], temperature=w.temperature, top_k=w.top_k,
                           top_p=w.top_p, penalty=w.penalty, seen_ids=h, u=b.uniforms[0])
    assert r["ids"][0] == want


@pytest.mark.parametrize("seed", range(6))
def test_small_random_rows_all_variants(oracle, seed):
    g = np.random.default_rng(seed)
    V = int(g.integers(2, 40))
    x = (g.standard_normal((1, V)) * g.uniform(0.5, 6)).astype(np.float32)
    if seed % 2:
        x[0, g.integers(0, V, 3)] = x[0, 0]  # ties
    hist = g.integers(0, V, 7).astype(np.uint32)
    off = np.array([0, hist.size], np.uint32)
    T = float(g.uniform(0.5, 1.5))
    k = int(g.integers(1, V + 3))
    tp = float(g.uniform(0.3, 0.99))
    pen = float(g.uniform(1.0, 3.0))
    u32 = np.array([g.uniform(0, 1)], np.float32)
    u64 = np.array([g.uniform(0, 1)])
    # qwen
    r = oracle.sample(oracle.make_params(oracle.QWEN, temperature=T, top_k=k, top_p=tp, penalty=pen),
                      x, off, hist, u32)
    if not r["flags"][0] & oracle.FLAG_TIE_CUT:
        assert r["ids"][0] == np_ref.qwen_row(x[0], temperature=T, top_k=k, top_p=tp, penalty=pen,
                                              seen_ids=hist, u=u32[0])
    # indextts
    r = oracle.sample(oracle.make_params(oracle.INDEXTTS, temperature=T, top_k=k, top_p=tp,
                                         penalty=pen), x, off, hist, u64)
    assert r["ids"][0] == np_ref.indextts_row(x[0], temperature=T, top_k=k, top_p=tp, penalty=pen,
                                              hist=hist, u=u64[0])
    # moss
    r = oracle.sample(oracle.make_params(oracle.MOSS, temperature=T, top_k=k, top_p=tp, penalty=pen),
                      x, off, hist, u64)
    if not r["flags"][0] & oracle.FLAG_TIE_CUT:
        assert r["ids"][0] == np_ref.moss_row(x[0], temperature=T, top_k=k, top_p=tp, penalty=pen,
                                              hist=hist, u=u64[0])
    # nano
    r = oracle.sample(oracle.make_params(oracle.MOSS_NANO, temperature=T, top_k=k, top_p=tp,
                                         penalty=pen), x, off, hist, u64)
    assert r["ids"][0] == np_ref.nano_row(x[0], temperature=T, top_k=k, top_p=tp, penalty=pen,
                                          hist=hist, u=u64[0])
    # cosyvoice3
    u2 = np.array([g.uniform(0, 1), g.uniform(0, 1)], np.float32)
    r = oracle.sample(oracle.make_params(oracle.COSY_RAS, top_k=k, top_p=tp, ras_win=5, ras_tau=0.2),
                      x, off, hist, u2)
    want, ras = np_ref.cosy_row(x[0], top_p=tp, top_k=k, win=5, tau=0.2, hist=hist, u0=u2[0], u1=u2[1])
    assert r["ids"][0] == want and bool(r["flags"][0] & oracle.FLAG_RAS) == ras


# ------------------------------------------------------------------ indextts beam-sample step
def _beam_kw(w):
    return dict(temperature=w.temperature, top_k=w.top_k, top_p=w.top_p, penalty=w.penalty, min_keep=2)


@pytest.mark.parametrize("first_step", [True, False])
def test_indextts_beam_step(oracle, first_step):
    # generation.rs:640-701: joint beam-major scores plus the beam score, six
    # draws without replacement, candidates by score descending
    w = synth.WORKLOADS["indextts-mel-256x8194"]
    bb = synth.make_beam_batch(w, 2, 3, first_step=first_step)
    p = oracle.make_params(oracle.INDEXTTS, **_beam_kw(w))
    r = oracle.idx_beam_step(p, bb.logits, bb.hist_off, bb.hist_ids, bb.beam_scores, 3, bb.uniforms, 6)
    for bi in range(2):
        rows = [bb.logits[bi * 3 + j] for j in range(3)]
        hists = [bb.hist_ids[bb.hist_off[bi * 3 + j]:bb.hist_off[bi * 3 + j + 1]] for j in range(3)]
        want = np_ref.indextts_beam_step(rows, hists, bb.beam_scores[bi * 3:bi * 3 + 3], 3,
                                         bb.uniforms[bi * 6:bi * 6 + 6], 6, **_beam_kw(w))
        assert r["status"][bi] == oracle.OK
        assert [(float(s), int(f)) for s, f in zip(r["scores"][bi], r["flat"][bi])] == want
        if first_step:
            # the active beam's kept set is drawn first; inactive beams refill the rest
            # (generation.rs:266-271)
            assert all(f < w.vocab for f in r["flat"][bi][:2])


def test_indextts_beam_step_one_beam_is_the_row_sampler(oracle):
    # one beam, one draw, beam score 0: the per-row sampler's id
    w = synth.WORKLOADS["indextts-mel-256x8194"]
    b = _rows(w, 6)
    p = oracle.make_params(oracle.INDEXTTS, **_beam_kw(w))
    r = oracle.sample(p, b.logits_f32, b.hist_off, b.hist_ids, b.uniforms)
    rb = oracle.idx_beam_step(p, b.logits_f32, b.hist_off, b.hist_ids, np.zeros(6), 1, b.uniforms, 1)
    assert np.array_equal(rb["flat"][:, 0], r["ids"])


def test_indextts_beam_step_too_few(oracle):
    # generation.rs:284-286: fewer finite joint scores than draws
    g = np.random.default_rng(3)
    x = (g.standard_normal((2, 50)) * 4).astype(np.float32)
    p = oracle.make_params(oracle.INDEXTTS, temperature=1.0, top_k=2, top_p=0.1, min_keep=2)
    r = oracle.idx_beam_step(p, x, None, None, np.zeros(2), 1, g.random(12), 6)
    assert list(r["status"]) == [oracle.ETOOFEW] * 2
    # two beams of two kept ids each, four draws: every kept id once
    r = oracle.idx_beam_step(p, x, None, None, np.zeros(2), 2, g.random(4), 4)
    k = oracle.sample(p, x, None, None, g.random(2), cap=8)
    want = sorted([j * 50 + int(i) for j in range(2) for i in k["keep_ids"][j][:k["keep_count"][j]]])
    assert r["status"][0] == oracle.OK and sorted(r["flat"][0].tolist()) == want
