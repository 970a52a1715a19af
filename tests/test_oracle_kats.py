"""Known-answer tests that pin the oracle to the reference's own unit tests.

Each test transcribes one reference test (cited) into the oracle's terms.
Where the reference asserts through a random stream the oracle cannot
reproduce (rand's StdRng), the assertion is restated for any uniform stream
and the reason is given.
"""
import math

import numpy as np
import pytest

NEG = -np.inf


def finite_ids(row):
    return [i for i, v in enumerate(np.asarray(row).ravel()) if np.isfinite(v)]


# --------------------------------------------------------------------- RNGs
def test_qwen_pcg_seed42_outputs(oracle):
    # PCG XSH RR outputs for seed 42 (integer arithmetic, sampling.rs:75-93):
    # 213896069, 1518578345, 893660385; rand_f32 = out as f32 / u32::MAX as f32.
    rng = oracle.QwenRng(42)
    for out in (213896069, 1518578345, 893660385):
        assert rng.rand_f32() == np.float32(out) / np.float32(4294967295.0)


def test_qwen_pcg_seeding_and_reset(oracle):
    # sampling.rs:707-757 (test_seeded_deterministic, test_reset, different seeds)
    a = [oracle.QwenRng(12345).rand_f32() for _ in range(1)]
    r1, r2 = oracle.QwenRng(12345), oracle.QwenRng(12345)
    v1 = [r1.rand_f32() for _ in range(10)]
    v2 = [r2.rand_f32() for _ in range(10)]
    assert v1 == v2 and a[0] == v1[0]
    r3 = oracle.QwenRng(67890)
    assert sum(x == y for x, y in zip(v1, [r3.rand_f32() for _ in range(10)])) < 10
    for x in v1:
        assert 0.0 <= x <= 1.0  # 1.0 is reachable (out >= 2^32 - 128)


def test_steprng_deterministic(oracle):
    # crates/cosyvoice3/src/rng.rs:224-232
    a, b = oracle.StepRng(42), oracle.StepRng(42)
    for _ in range(8):
        assert a.next_u32() == b.next_u32()
    assert oracle.StepRng(42).next_u32() != oracle.StepRng(43).next_u32()


def test_steprng_closed_form(oracle):
    # rng.rs:158-180 restated in Python integers
    M = (1 << 64) - 1

    def step(state, inc):
        old = state
        state = (old * 6364136223846793005 + inc) & M
        xs = (((old >> 18) ^ old) >> 27) & 0xFFFFFFFF
        rot = old >> 59
        return state, ((xs >> rot) | (xs << ((32 - rot) & 31))) & 0xFFFFFFFF

    for seed in (0, 7, 42, 2**63 + 5):
        inc = ((seed << 1) | 1) & M
        st, _ = step(0, inc)
        st = (st + 0x853C49E6748FEA9D) & M
        st, _ = step(st, inc)
        r = oracle.StepRng(seed)
        for _ in range(5):
            st, out = step(st, inc)
            assert r.next_u32() == out


def test_nano_lcg_first_draw(oracle):
    # nano/sampling.rs:85-86: "Seed 42's first LCG draw is 0.252345..."
    u = oracle.NanoLcg(42).next_unit()
    assert abs(u - 0.252345) < 1e-6
    assert u == ((42 * 1664525 + 1013904223) % 2**32 >> 8) / 16777216.0


# --------------------------------------------------------------------- qwen
def test_greedy_sample(oracle):
    # sampling.rs:468-491
    assert oracle.argmax([1.0, 2.0, 5.0, 1.0]) == 2
    for row, want in (([1.0, 5.0, 2.0], 1), ([3.0, 1.0, 2.0], 0), ([1.0, 2.0, 10.0], 2)):
        assert oracle.argmax(row) == want


def _qwen_sample(oracle, logits, seed, **kw):
    logits = np.asarray(logits, np.float32)
    rows = logits.shape[0]
    rng = oracle.QwenRng(seed)
    p = oracle.make_params(oracle.QWEN, **kw)
    greedy = kw.get("temperature", 1.0) < 0.01
    u = np.array([0.0 if greedy else rng.rand_f32() for _ in range(rows)], np.float32)
    return oracle.sample(p, logits, uniforms=u)["ids"].tolist()


def test_sample_very_low_temperature_and_batch(oracle):
    # sampling.rs:493-506 and 692-705 (T = 0.001 takes greedy)
    assert _qwen_sample(oracle, [[1.0, 10.0, 2.0, 1.0]], 42, temperature=0.001, top_k=50,
                        top_p=0.9) == [1]
    assert _qwen_sample(oracle, [[10.0, 1.0, 1.0], [1.0, 10.0, 1.0]], 42, temperature=0.001,
                        top_k=50, top_p=0.9) == [0, 1]


def test_qwen_repetition_penalty(oracle):
    # sampling.rs:535-574, 677-690, 983-995
    x = oracle.qwen_penalty_ids([[1.0, 2.0, 3.0]], [0], 1.0)
    assert x.tolist() == [[1.0, 2.0, 3.0]]
    assert oracle.qwen_penalty_ids([[2.0, 3.0, 4.0]], [0], 2.0).tolist() == [[1.0, 3.0, 4.0]]
    assert oracle.qwen_penalty_ids([[-2.0, 3.0, 4.0]], [0], 2.0)[0, 0] == -4.0
    assert oracle.qwen_penalty_ids([[2.0, 3.0, 4.0, 5.0]], [0, 2], 2.0).tolist() == [[1.0, 3.0, 2.0, 5.0]]
    logits = [[2.0, -4.0, 6.0], [-2.0, 4.0, -6.0]]
    a = oracle.qwen_penalty_ids(logits, [0, 1], 2.0)
    b = oracle.qwen_penalty_mask(logits, [1.0, 1.0, 0.0], 2.0)
    assert a.tolist() == b.tolist() == [[1.0, -8.0, 6.0], [-4.0, 2.0, -6.0]]
    # ids >= V are ignored, duplicates idempotent (sampling.rs:349-353)
    assert oracle.qwen_penalty_ids([[2.0, 3.0]], [1, 1, 7], 2.0).tolist() == [[2.0, 1.5]]


def test_qwen_penalty_is_reciprocal_multiply(oracle):
    # sampling.rs:388-395: positive logits are multiplied by f32(1/pen), not divided.
    pen = 1.1
    inv = np.float32(1.0) / np.float32(pen)
    xs = np.array([[0.7, 3.3, 9.1, 12.345]], np.float32)
    got = oracle.qwen_penalty_ids(xs, [0, 1, 2, 3], pen)
    assert np.array_equal(got, xs * inv)
    assert not np.array_equal(got, xs / np.float32(pen))


def test_multinomial_deterministic_probs(oracle):
    # sampling.rs:595-604
    rng = oracle.QwenRng(42)
    assert oracle.first_cdf_index([0.0, 1.0, 0.0, 0.0], rng.rand_f32()) == 1


def test_first_cdf_index_boundaries(oracle):
    # sampling.rs:606-621
    row = [0.25, 0.5, 0.25]
    for thr, want in ((0.0, 0), (0.25, 0), (0.250001, 1), (0.75, 1), (0.750001, 2), (1.0, 2)):
        assert oracle.first_cdf_index(row, thr) == want
    assert oracle.first_cdf_index([0.0] * 4, 0.5) is None
    assert oracle.first_cdf_index([np.nan, 0.5], 0.25) is None


def _legacy_choice(cdf, thr):
    # the legacy tensor rule: first position with cdf >= thr, else argmin of all-5 -> 0
    for i, v in enumerate(cdf):
        if v >= thr:
            return i
    return 0


def test_multinomial_fallback_matches_legacy(oracle):
    # sampling.rs:623-641 (rows of zeros, NaN and 0.01)
    for row in ([0.0] * 4, [np.nan] * 4, [0.01] * 4):
        r = np.asarray(row, np.float32)
        thr = oracle.QwenRng(42).rand_f32()
        cdf = np.cumsum(r.astype(np.float64)).astype(np.float32)
        i = oracle.first_cdf_index(r, thr)
        assert (0 if i is None else i) == _legacy_choice(cdf, thr)


def test_multinomial_dyadic_fixture(oracle):
    # sampling.rs:643-675: dyadic probabilities keep every accumulation exact,
    # so the legacy cumsum is the exact prefix sum.
    for vocab in (4, 3072):
        rows = []
        for batch in range(2):
            row = [((i * 37 + batch * 17) % 5) / 16384.0 for i in range(vocab - 1)]
            row.append(1.0 - float(np.float32(sum(row))))
            rows.append(np.asarray(row, np.float32))
        cdfs = [np.cumsum(r.astype(np.float64)) for r in rows]
        for seed in range(512):
            rng = oracle.QwenRng(seed)
            for r, cdf in zip(rows, cdfs):
                thr = rng.rand_f32()
                i = oracle.first_cdf_index(r, thr)
                assert (0 if i is None else i) == _legacy_choice(cdf, float(thr)), (vocab, seed)


def test_top_k_then_top_p_original_ids(oracle):
    # sampling.rs:789-804
    row, _ = oracle.qwen_top_k([1.0, 5.0, 3.0, 2.0, 4.0, 4.0], 3)
    assert finite_ids(row) == [1, 4, 5]
    row, _ = oracle.qwen_top_p(row, 0.9)
    assert finite_ids(row) == [1, 4, 5]


def test_nucleus_boundaries(oracle):
    # sampling.rs:818-853 (check_nucleus_boundaries)
    sparse = np.full(3072, NEG, np.float32)
    for i, v in ((1001, 4.0), (500, 3.0), (2000, 2.0), (100, 1.0)):
        sparse[i] = v
    assert finite_ids(oracle.qwen_top_p(sparse, 0.8)[0]) == [500, 1001]
    kept = finite_ids(oracle.qwen_top_p([2.0, 1.0, 1.0, -10.0], 0.7)[0])
    assert len(kept) == 2 and 0 in kept and all(i < 3 for i in kept)
    # uniform p = 0.5: cumulative 0.25, 0.5, 0.75 -> "equal to p is not exceeding"
    assert len(finite_ids(oracle.qwen_top_p([0.0] * 4, 0.5)[0])) == 3
    a = oracle.qwen_top_p([0.0, 3.0, 1.0, 2.0], 0.6)[0]
    b = oracle.qwen_top_p([2.0, 1.0, 3.0, 0.0], 0.6)[0]
    assert np.isfinite(a[1]) and np.isfinite(b[2])
    assert len(finite_ids(a)) + len(finite_ids(b)) == 2


def test_top_k_matches_sort_at_model_vocab(oracle):
    # sampling.rs:902-931
    rows = []
    for offset in range(4):
        rows.append(np.array([NEG if (i + offset) % 17 == 0 else ((i * 37 + offset) % 101) - 50.0
                              for i in range(3072)], np.float32))
    for k in (1, 2, 50, 1024, 3072, 4096):
        for row in rows:
            got, _ = oracle.qwen_top_k(row, k)
            thr = np.sort(row)[::-1][min(k, row.size) - 1]
            want = np.where(row >= thr, row, NEG).astype(np.float32)
            assert np.array_equal(got, want), k


def test_top_k_filter_cases(oracle):
    # sampling.rs:933-957
    v, _ = oracle.qwen_top_k([1.0, 5.0, 3.0, 2.0, 4.0], 3)
    assert v[1] == 5.0 and v[4] == 4.0 and v[2] == 3.0 and v[0] == NEG and v[3] == NEG
    v, _ = oracle.qwen_top_k([1.0, 2.0, 3.0], 100)
    assert v.tolist() == [1.0, 2.0, 3.0]


def test_top_p_filter_cases(oracle):
    # sampling.rs:959-981
    v, _ = oracle.qwen_top_p([10.0, 0.0, 0.0, 0.0], 0.9)
    assert v[0] == 10.0
    v, _ = oracle.qwen_top_p([1.0, 1.0, 1.0, 1.0], 0.5)
    assert 2 <= int(np.isfinite(v).sum()) <= 4


def test_suppression_mask(oracle):
    # tts.rs:72-166
    m = oracle.qwen_suppression_mask(3072, 2150)
    x = oracle.qwen_add_mask(np.ones((3, 3072), np.float32), m)
    for r in range(3):
        assert x[r, 0] == 1.0 and x[r, 2047] == 1.0
        assert x[r, 2048] == NEG and x[r, 2149] == NEG and x[r, 2151] == NEG and x[r, 3071] == NEG
        assert x[r, 2150] == 1.0


def test_device_parity_template_rows_are_stable(oracle):
    # sampling.rs:873-900 run twice through the oracle: the same seed gives the
    # same ids (determinism of the seeded pipeline).
    for vocab in (4, 3072):
        row = np.full(vocab, NEG, np.float32)
        for i, v in ((vocab - 1, 2.0), (vocab // 2, 1.0), (1, 1.0)):
            row[i] = v
        for top_p in (0.5, 0.7, 0.9):
            for seed in range(16):
                a = _qwen_sample(oracle, [row], seed, temperature=0.7, top_k=3, top_p=top_p)
                b = _qwen_sample(oracle, [row], seed, temperature=0.7, top_k=3, top_p=top_p)
                assert a == b and a[0] in (1, vocab // 2, vocab - 1)


# --------------------------------------------------------------------- indextts
def test_indextts_repetition_penalty(oracle):
    # generation.rs:803-817
    assert oracle.idx_penalty([-2.0, 3.0, -0.5, 1.0], [0, 1, 3], 2.0).tolist() == [-4.0, 1.5, -0.5, 0.5]
    assert oracle.idx_penalty([-2.0, -3.0], [0], 10.0).tolist() == [-20.0, -3.0]
    assert oracle.idx_penalty([4.0, 1.0], [0, 0], 2.0).tolist() == [2.0, 1.0]


def test_indextts_top_k_ties(oracle):
    # generation.rs:819-841
    assert oracle.idx_top_k([1.0, 4.0, 4.0, 2.0, 3.0], 2).tolist() == [NEG, 4.0, 4.0, NEG, NEG]
    assert oracle.idx_top_k([5.0, 4.0, 1.0, 1.0], 1).tolist() == [5.0, 4.0, NEG, NEG]
    v = oracle.idx_top_k([5.0, 1.0, 2.0], 2)
    assert v[2] == 2.0 and v[1] == NEG


def test_indextts_top_p_mass_boundary(oracle):
    # generation.rs:843-868
    ln = lambda v: float(np.log(np.float32(v)))  # noqa: E731  (f32 ln)
    s = oracle.idx_top_p([ln(0.5), ln(0.3), ln(0.2)], 0.5)
    assert np.isfinite(s[0]) and np.isfinite(s[1]) and s[2] == NEG
    s = oracle.idx_top_p([ln(0.55), ln(0.25), ln(0.15), ln(0.05)], 0.85)
    assert np.isfinite(s[:3]).all() and s[3] == NEG
    s = oracle.idx_top_p([ln(0.6), ln(0.25), ln(0.15)], 0.9)
    assert np.isfinite(s).all()


def test_indextts_typical(oracle):
    # generation.rs:870-882
    ln = lambda v: float(np.log(np.float32(v)))  # noqa: E731
    s = oracle.idx_typical([ln(0.5), ln(0.3), ln(0.2)], 0.5)
    assert np.isfinite(s[0]) and np.isfinite(s[1]) and s[2] == NEG


def test_indextts_inverse_cdf(oracle):
    # generation.rs:884-895
    w = [0.2, 0.5, 0.3]
    for u, want in ((0.1, 0), (0.2, 1), (0.69, 1), (0.7, 2), (0.999, 2)):
        assert oracle.idx_inverse_cdf(w, u) == want
    assert oracle.idx_inverse_cdf([0.0, 0.5, 0.5], 0.1) == 1


def test_indextts_concentrated_refill(oracle):
    # generation.rs:917-935: the first two picks are [0, 1] for every uniform
    # stream (weights are exactly 1.0 then exactly 1.0 after removal), which is
    # why the StdRng stream of the reference test does not matter here.
    scores = [0.0, -40.0, -1e9, -1e9 - 40.0, -1e9, -1e9 - 40.0]
    for us in ([0.0] * 6, [0.999999] * 6, np.linspace(0.01, 0.99, 6)):
        picks = oracle.idx_sample_wo_replacement(scores, 6, us)
        assert picks[:2] == [0, 1] and len(set(picks)) == 6


def test_indextts_without_replacement_mass(oracle):
    # generation.rs:897-915 with a PCG64 uniform stream in place of StdRng
    scores = np.log(np.array([0.05, 0.05, 0.8, 0.05, 0.05]))
    g = np.random.Generator(np.random.PCG64(294738))
    us = g.random(3)
    a = oracle.idx_sample_wo_replacement(scores, 3, us)
    assert a == oracle.idx_sample_wo_replacement(scores, 3, us) and len(set(a)) == 3
    g = np.random.Generator(np.random.PCG64(7))
    firsts = [0] * 5
    for _ in range(400):
        firsts[oracle.idx_sample_wo_replacement(scores, 1, g.random(1))[0]] += 1
    assert firsts[2] > 300


def test_indextts_too_few_candidates(oracle):
    # generation.rs:284-286
    assert oracle.idx_sample_wo_replacement([NEG, NEG, 0.0], 2, [0.5, 0.5]) is None


def test_indextts_log_softmax(oracle):
    # generation.rs:948-960
    row = oracle.idx_log_softmax([1.0, 2.0, 3.0])
    e = np.float32
    s = e(math.exp(0.0)) + e(np.exp(e(-1.0))) + e(np.exp(e(-2.0)))
    for a, x in zip(row, (-2.0, -1.0, 0.0)):
        assert abs(a - (x - np.log(s))) < 1e-6


# --------------------------------------------------------------------- cosyvoice3
def test_cosy_nucleus_respects_top_k(oracle):
    # llm.rs:699-711
    probs = oracle.softmax([0.1, 10.0, 9.0, 0.1, 0.1])
    rng = oracle.StepRng(7)
    for _ in range(64):
        t, used, _ = oracle.cosy_nucleus(probs, 0.9, 2, rng.next_f32())
        assert used and t in (1, 2)


def test_cosy_ignore_eos(oracle):
    # llm.rs:713-735: speech_token_size 6561, vocab 6761
    vocab, eos = 6761, 6561
    raw = np.full((1, vocab), -20.0, np.float32)
    raw[0, eos] = 50.0
    raw[0, 7] = 10.0
    rng = oracle.StepRng(42)
    kw = dict(top_p=0.9, top_k=5, ras_win=10, ras_tau=0.1)
    p = oracle.make_params(oracle.COSY_RAS, eos_id=eos, **kw)
    u = np.array([rng.next_f32(), 0.0], np.float32)
    r = oracle.sample(p, raw, np.array([0, 0], np.uint32), np.zeros(0, np.uint32), u)
    assert r["ids"][0] == 7
    p = oracle.make_params(oracle.COSY_RAS, eos_id=-1, **kw)
    u = np.array([rng.next_f32(), 0.0], np.float32)
    r = oracle.sample(p, raw, np.array([0, 0], np.uint32), np.zeros(0, np.uint32), u)
    assert r["ids"][0] == eos


def test_cosy_invalid_params(oracle):
    # llm.rs:436-445
    x = np.zeros((1, 4), np.float32)
    u = np.zeros(2, np.float32)
    for bad in (dict(top_p=0.0), dict(top_p=1.5), dict(top_k=0), dict(ras_win=0),
                dict(ras_tau=2.0), dict(top_p=float("nan"))):
        kw = dict(top_p=0.8, top_k=25, ras_win=10, ras_tau=0.1)
        kw.update(bad)
        r = oracle.sample(oracle.make_params(oracle.COSY_RAS, **kw), x, np.array([0, 0], np.uint32),
                          np.zeros(0, np.uint32), u)
        assert r["rc"] == oracle.EINVAL


def test_cosy_ras_fallback_fires_on_repeat(oracle):
    # llm.rs:532-536: one repeat of the nucleus token in the last 10 fires RAS
    x = np.zeros((1, 8), np.float32)
    x[0, 3] = 30.0  # nucleus token is 3 for any u0
    kw = dict(top_p=0.8, top_k=25, ras_win=10, ras_tau=0.1)
    u = np.array([0.5, 0.999], np.float32)
    hist = np.array([3, 1, 1], np.uint32)
    r = oracle.sample(oracle.make_params(oracle.COSY_RAS, **kw), x, np.array([0, 3], np.uint32), hist, u)
    assert r["flags"][0] & oracle.FLAG_RAS and r["ids"][0] == 3  # fallback CDF over all V
    hist = np.array([3] + [1] * 10, np.uint32)  # the 3 is outside the window of 10
    r = oracle.sample(oracle.make_params(oracle.COSY_RAS, **kw), x, np.array([0, 11], np.uint32), hist, u)
    assert not (r["flags"][0] & oracle.FLAG_RAS) and r["ids"][0] == 3


# --------------------------------------------------------------------- moss-nano
def _nano(oracle, logits, hist, T, k, p, pen, seed=42):
    x = np.asarray([logits], np.float32)
    u = np.array([oracle.NanoLcg(seed).next_unit()], np.float64)
    hist = np.asarray(hist, np.uint32)
    prm = oracle.make_params(oracle.MOSS_NANO, temperature=T, top_k=k, top_p=p, penalty=pen)
    r = oracle.sample(prm, x, np.array([0, hist.size], np.uint32), hist, u)
    return int(r["ids"][0]), int(r["status"][0])


def test_nano_fixed_draws(oracle):
    # nano/sampling.rs:82-99
    assert _nano(oracle, [0.0, 1.0, 2.0, 3.0], [], 1.0, 4, 1.0, 1.0) == (2, 0)
    assert _nano(oracle, [0.0, 1.0, 2.0, 3.0], [], 1.0, 4, 0.5, 1.0) == (3, 0)
    assert _nano(oracle, [0.0, 1.0, 2.0, 3.0], [3, 3, 3], 1.0, 1, 1.0, 2.0) == (2, 0)
    assert _nano(oracle, [np.nan], [], 1.0, 1, 1.0, 1.0)[1] == oracle.ENONFINITE
    assert _nano(oracle, [0.0, 1.0], [5], 1.0, 1, 1.0, 2.0)[1] == oracle.EINVAL


# --------------------------------------------------------------------- moss
def test_moss_errors_and_greedy(oracle):
    # moss-tts/src/sampling.rs:48-59
    x = np.array([[0.0, np.nan, 1.0]], np.float32)
    prm = oracle.make_params(oracle.MOSS, temperature=0.8, top_k=30, top_p=0.6, penalty=1.1)
    r = oracle.sample(prm, x, np.array([0, 0], np.uint32), np.zeros(0, np.uint32), np.array([0.5]))
    assert r["status"][0] == oracle.ENONFINITE
    x = np.array([[0.0, 2.0, 1.0]], np.float32)
    prm = oracle.make_params(oracle.MOSS, temperature=0.0, top_k=30, top_p=0.6, penalty=1.0)
    r = oracle.sample(prm, x, np.array([0, 0], np.uint32), np.zeros(0, np.uint32), np.array([0.5]))
    assert r["ids"][0] == 1
    prm = oracle.make_params(oracle.MOSS, temperature=0.8, top_k=30, top_p=0.6, penalty=1.0,
                             exclude_id=1)
    r = oracle.sample(prm, x, np.array([0, 0], np.uint32), np.zeros(0, np.uint32), np.array([0.99]))
    assert r["ids"][0] in (0, 2)


# --------------------------------------------------------------------- indextts beam search (do_sample = false)
def _processed(oracle, row, hist, pen):
    r = oracle.idx_log_softmax(row)
    return oracle.idx_penalty(r, hist, pen) if pen != 1.0 else r


def test_indextts_beam_search_selects_best_joint_scores(oracle):
    # generation.rs:671-679: every flat index sorted by joint score descending
    # (a stable sort: equal scores in ascending flat order), truncated to
    # n_keep.  Checked against numpy's stable argsort of the joint scores the
    # oracle's own (pinned) processors give.
    g = np.random.default_rng(9)
    nb, V, n_keep = 3, 257, 6
    x = (g.standard_normal((2 * nb, V)) * 3).astype(np.float32)
    x[1] = x[0]                      # a beam equal to beam 0: every score tied across them
    bonus = np.array([0.0, 0.0, -1e9, -0.5, -1.25, -3.0])
    hist = [g.integers(0, V, 40).astype(np.uint32) for _ in range(2 * nb)]
    hist[1] = hist[0]                # and the same history
    off = np.zeros(2 * nb + 1, np.uint32)
    off[1:] = np.cumsum([h.size for h in hist])
    prm = oracle.make_params(oracle.INDEXTTS, temperature=0.7, top_k=5, top_p=0.5, penalty=1.7)
    r = oracle.idx_beam_search_step(prm, x, off, np.concatenate(hist), bonus, nb, n_keep)
    for bi in range(2):
        joint = np.concatenate([_processed(oracle, x[bi * nb + j], hist[bi * nb + j], 1.7).astype(np.float64)
                                + bonus[bi * nb + j] for j in range(nb)])
        want = np.argsort(-joint, kind="stable")[:n_keep]
        assert r["flat"][bi].tolist() == want.tolist()
        assert r["scores"][bi].tolist() == joint[want].tolist()
    # element 0: beams 0 and 1 tie everywhere, so each pair of candidates is
    # (beam 0 id, beam 1 id) for the same id, beam 0 first
    f = r["flat"][0]
    assert [int(v) // V for v in f] == [0, 1] * (n_keep // 2)
    assert all(int(f[i]) % V == int(f[i + 1]) % V for i in range(0, n_keep, 2))


def test_indextts_beam_search_skips_the_sampling_warpers(oracle):
    # temperature, top-k and top-p apply only when sampling (generation.rs:653-662):
    # the joint scores are the log-probs with the penalty, whatever they are set to
    g = np.random.default_rng(10)
    V = 100
    x = (g.standard_normal((1, V)) * 2).astype(np.float32)
    a = oracle.idx_beam_search_step(oracle.make_params(oracle.INDEXTTS, temperature=0.3, top_k=2, top_p=0.1),
                                    x, None, None, np.zeros(1), 1, 8)
    b = oracle.idx_beam_search_step(oracle.make_params(oracle.INDEXTTS), x, None, None, np.zeros(1), 1, 8)
    assert a["flat"].tolist() == b["flat"].tolist() and a["scores"].tolist() == b["scores"].tolist()
    ls = oracle.idx_log_softmax(x[0]).astype(np.float64)
    assert a["scores"][0].tolist() == np.sort(ls)[::-1][:8].tolist()
