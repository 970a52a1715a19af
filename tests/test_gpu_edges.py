"""Edge cases and reference known-answer rows through the HIP sampler, each
checked against the oracle on identical inputs (ties, -inf/NaN/+inf rows, k
larger than V, greedy, misaligned and padded rows, bf16, penalty modes,
suppression and EOS masks, error statuses)."""
import numpy as np
import pytest

torch = pytest.importorskip("torch")

from oracle import oracle as O  # noqa: E402
from talechime_amd import _lib  # noqa: E402
from talechime_amd.sampler import DeviceSampler, make_params  # noqa: E402

pytestmark = pytest.mark.gpu
NEG = -np.inf
CAP = 64
KSURV = 1024  # survivors the kernels stage in LDS


@pytest.fixture(scope="module")
def sampler():
    if not torch.cuda.is_available():
        pytest.skip("no GPU visible")
    s = DeviceSampler(0, max_rows=4096, max_vocab=1 << 18)
    yield s
    s.close()


def run(sampler, variant, logits, hist=None, uniforms=None, *, ld_pad=0, bf16=False,
        hist_mode=0, add_mask=None, pen_mask=None, **kw):
    """Sample with both the GPU and the oracle; returns (gpu dict, oracle dict)."""
    x = np.ascontiguousarray(logits, np.float32)
    rows, V = x.shape
    if hist is None:
        hist = [[] for _ in range(rows)]
    if hist_mode == 1:
        off = np.array([0, len(hist[0])], np.uint32)
        ids = np.asarray(hist[0], np.uint32)
    else:
        off = np.zeros(rows + 1, np.uint32)
        off[1:] = np.cumsum([len(h) for h in hist])
        ids = np.concatenate([np.asarray(h, np.uint32) for h in hist]) if off[-1] else np.zeros(0, np.uint32)
    f64 = variant in (O.INDEXTTS, O.MOSS, O.MOSS_NANO)
    per = 2 if variant == O.COSY_RAS else 1
    u = np.asarray(uniforms, np.float64 if f64 else np.float32).reshape(-1)
    assert u.size >= rows * per
    # device copy, optionally padded rows (ld > V) and bf16
    ld = V + ld_pad
    if bf16:
        bits = np.zeros((rows, ld), np.uint16)
        from talechime_amd.synth import bf16_bits_to_f32, to_bf16_bits
        bits[:, :V] = to_bf16_bits(x)
        x = bf16_bits_to_f32(bits[:, :V]).copy()
        dl = torch.from_numpy(bits.view(np.int16)).view(torch.bfloat16).cuda()[:, :V]
    else:
        buf = np.zeros((rows, ld), np.float32)
        buf[:, :V] = x
        dl = torch.from_numpy(buf).cuda()[:, :V]
    dho = torch.from_numpy(off.view(np.int32).copy()).cuda()
    dhi = torch.from_numpy((ids if ids.size else np.zeros(1, np.uint32)).view(np.int32).copy()).cuda()
    du = torch.from_numpy(u).cuda()
    am = torch.from_numpy(np.asarray(add_mask, np.float32)).cuda() if add_mask is not None else None
    pm = torch.from_numpy(np.asarray(pen_mask, np.float32)).cuda() if pen_mask is not None else None
    p = make_params(variant, hist_mode=hist_mode, add_mask=am, pen_mask=pm, **kw)
    r = sampler.sample(p, dl, dho, dhi, du, verify_cap=CAP)
    torch.cuda.synchronize()
    g = {k: getattr(r, k).cpu().numpy() for k in ("ids", "status", "flags", "topk_count", "topk_ids",
                                                  "keep_count", "keep_ids", "keep_probs", "norm")}
    g["ids"] = g["ids"].view(np.uint32)
    if variant in (O.INDEXTTS, O.QWEN, O.COSY_RAS):
        # without verification outputs the indextts, qwen and cosyvoice3
        # kernels decide from approximate sums first: the same ids, statuses
        # and flags (indextts rows near a tie of the f64 decisions aside)
        r0 = sampler.sample(p, dl, dho, dhi, du, verify_cap=0)
        torch.cuda.synchronize()
        ids0, st0 = r0.ids.cpu().numpy().view(np.uint32), r0.status.cpu().numpy()
        keep = (g["flags"] & 16) == 0
        assert np.array_equal(st0, g["status"])
        assert np.array_equal(ids0[keep], g["ids"][keep]), np.nonzero(ids0 != g["ids"])[0][:10]
        if variant in (O.QWEN, O.COSY_RAS):
            assert np.array_equal(r0.flags.cpu().numpy(), g["flags"])
    okw = dict(kw)
    okw["penalty"] = okw.pop("penalty", 1.0)
    op = O.make_params(variant, hist_mode=hist_mode, add_mask=add_mask, pen_mask=pen_mask, **okw)
    o = O.sample(op, x, off, ids, u, cap=CAP)
    return g, o


def same(g, o, rows=None, probs_exact=True):
    rows = range(g["ids"].size) if rows is None else rows
    for r in rows:
        if o["status"][r] != 0:
            assert g["status"][r] == o["status"][r], (r, g["status"][r], o["status"][r])
            continue
        assert g["status"][r] == 0, (r, g["status"][r])
        assert g["ids"][r] == o["ids"][r], (r, g["ids"][r], o["ids"][r])
        # TC_FLAG_NEAR_TIE (16) reports a decision within the f64 exp error of the
        # reference's libm; the oracle has no such flag
        assert g["flags"][r] & ~16 == o["flags"][r], (r, g["flags"][r], o["flags"][r])
        for c, i in (("topk_count", "topk_ids"), ("keep_count", "keep_ids")):
            assert g[c][r] == o[c][r], (r, c, g[c][r], o[c][r])
            n = min(int(g[c][r]), CAP)
            assert np.array_equal(g[i][r, :n].astype(np.uint32), o[i][r, :n]), (r, i)
        assert np.array_equal(g["norm"][r:r + 1], o["norm"][r:r + 1], equal_nan=True), (r, g["norm"][r], o["norm"][r])
        n = min(int(g["keep_count"][r]), CAP)
        if probs_exact:
            assert np.array_equal(g["keep_probs"][r, :n], o["keep_probs"][r, :n], equal_nan=True), r
        else:
            np.testing.assert_allclose(g["keep_probs"][r, :n], o["keep_probs"][r, :n], rtol=1e-5)


QWEN_KW = dict(temperature=0.7, top_k=50, top_p=0.9)


# ------------------------------------------------------------------ qwen
@pytest.mark.parametrize("vocab", [4, 3072])
def test_qwen_device_parity_template(sampler, vocab):
    # crates/qwen3-tts/src/generation/sampling.rs:873-900
    row = np.full(vocab, NEG, np.float32)
    for i, v in ((vocab - 1, 2.0), (vocab // 2, 1.0), (1, 1.0)):
        row[i] = v
    for top_p in (0.5, 0.7, 0.9):
        for seed in range(16):
            u = [O.QwenRng(seed).rand_f32()]
            g, o = run(sampler, O.QWEN, [row], uniforms=u, temperature=0.7, top_k=3, top_p=top_p)
            same(g, o)


def test_qwen_reference_rows(sampler):
    # sampling.rs:493-506, 692-705 (greedy), 789-804, 818-848
    g, o = run(sampler, O.QWEN, [[1.0, 10.0, 2.0, 1.0]], uniforms=[0.3], temperature=0.001, top_k=50, top_p=0.9)
    assert g["ids"][0] == 1 and g["flags"][0] == _lib.FLAG_GREEDY
    g, o = run(sampler, O.QWEN, [[10.0, 1.0, 1.0], [1.0, 10.0, 1.0]], uniforms=[0.3, 0.3], temperature=0.001,
               top_k=50, top_p=0.9)
    assert g["ids"].tolist() == [0, 1]
    g, o = run(sampler, O.QWEN, [[1.0, 5.0, 3.0, 2.0, 4.0, 4.0]], uniforms=[0.99], temperature=1.0, top_k=3,
               top_p=0.9)
    same(g, o)
    assert sorted(g["topk_ids"][0, :3].tolist()) == [1, 4, 5]
    sparse = np.full(3072, NEG, np.float32)
    for i, v in ((1001, 4.0), (500, 3.0), (2000, 2.0), (100, 1.0)):
        sparse[i] = v
    g, o = run(sampler, O.QWEN, [sparse], uniforms=[0.5], temperature=1.0, top_k=0, top_p=0.8)
    same(g, o)
    assert g["keep_ids"][0, :2].tolist() == [500, 1001]


def test_qwen_fast_path_and_fallback_distributions(sampler):
    """Rows the qwen fast path stages (peaked scores) and rows it hands to the
    general path (flat scores: more than 128 candidates near the k-th; -inf
    entries; k above 64), each bit-exact against the oracle with the
    verification outputs."""
    g_ = np.random.default_rng(77)
    for V in (2048, 3072):
        rows = []
        for sigma in (0.05, 0.5, 2.0, 6.0, 20.0):
            rows.append((g_.standard_normal(V) * sigma).astype(np.float32))
        masked = (g_.standard_normal(V) * 3).astype(np.float32)
        masked[g_.integers(0, V, V // 3)] = NEG
        rows.append(masked)
        x = np.stack(rows)
        n = len(rows)
        hist = [g_.integers(0, V, 80).tolist() for _ in range(n)]
        u = [O.QwenRng(V + r).rand_f32() for r in range(n)]
        for k, p in ((1, 0.9), (2, 0.5), (50, 0.8), (64, 1.0), (65, 0.9), (200, 0.7)):
            g, o = run(sampler, O.QWEN, x, hist, u, temperature=0.9, top_k=k, top_p=p, penalty=1.2)
            tie = (o["flags"] & 1) != 0
            same(g, o, rows=[r for r in range(n) if not tie[r]])


def test_qwen_many_survivors_without_top_p(sampler):
    """top-k off (or wider than 1024) and top-p off: softmax and CDF over every
    survivor of the register-resident row, bit-exact with the verification
    outputs; with top-p on, every survivor goes through the rank sort."""
    g_ = np.random.default_rng(31)
    for V in (3072, 8194, 16000):
        x = (g_.standard_normal((6, V)) * 2).astype(np.float32)
        x[1, g_.integers(0, V, V // 4)] = NEG
        x[2, :] = 0.0                                    # every probability equal
        x[3, : V // 2] = NEG
        hist = [g_.integers(0, V, 64).tolist() for _ in range(6)]
        u = [0.0, 0.25, 0.5, 0.999999, 1.0, O.QwenRng(V).rand_f32()]
        for k in (0, 5000, V + 3):
            g, o = run(sampler, O.QWEN, x, hist, u, temperature=0.8, top_k=k, top_p=1.0, penalty=1.1)
            same(g, o)
        for tp in (0.9, 0.3):
            g, o = run(sampler, O.QWEN, x, hist, u, temperature=0.8, top_k=0, top_p=tp, penalty=1.1)
            assert (g["status"] == 0).all(), g["status"]
            tie = (o["flags"] & 1) != 0
            same(g, o, rows=np.nonzero(~tie)[0])
            assert np.array_equal(g["flags"], o["flags"].astype(np.int32))


@pytest.mark.parametrize("V,k", [(3072, 0), (2048, 0), (4096, 2000), (3072, 3072), (8194, 0), (16384, 0),
                                 (12000, 9000)])
def test_qwen_top_p_over_many_survivors(sampler, V, k):
    # top-k off or wide, top-p on: every survivor sorted into rank order, the
    # denominator and the running sum as the reference's sequential f32 sums
    g_ = np.random.default_rng(V + k)
    rows = 10
    x = (g_.standard_normal((rows, V)) * 1.5).astype(np.float32)
    x[1, g_.integers(0, V, V // 3)] = NEG
    x[2] = np.round(x[2] * 2) / 2  # many equal values
    hist = [g_.integers(0, V, 64).tolist() for _ in range(rows)]
    u = g_.random(rows).astype(np.float32)
    for tp in (0.5, 0.9, 0.99):
        g, o = run(sampler, O.QWEN, x, hist, u, temperature=0.9, top_k=k, top_p=tp, penalty=1.1)
        assert (o["topk_count"] > 1024).any()
        tie = (o["flags"] & 1) != 0
        same(g, o, rows=np.nonzero(~tie)[0])
        assert np.array_equal(g["flags"], o["flags"].astype(np.int32))


def test_qwen_ties_and_degenerate_rows(sampler):
    rows = [
        np.zeros(64, np.float32),                     # all equal: ties at top-k and top-p
        np.full(64, NEG, np.float32),                 # all -inf -> index 0
        np.r_[np.float32(np.inf), np.zeros(63, np.float32)],  # +inf -> NaN CDF -> index 0
        np.arange(64, dtype=np.float32) % 4,          # repeated values
    ]
    for u in (0.0, 0.37, 1.0):
        for k, p in ((5, 0.5), (64, 0.95), (100, 0.3), (1, 0.9), (0, 0.6)):
            g, o = run(sampler, O.QWEN, rows, uniforms=[u] * 4, temperature=1.0, top_k=k, top_p=p)
            tie = (o["flags"] & 1) != 0
            same(g, o, rows=[r for r in range(4) if not tie[r]])


def test_qwen_greedy_nan_and_ties(sampler):
    rows = np.array([[np.nan, 5.0, 5.0, 1.0], [1.0, 5.0, 5.0, np.nan], [-0.0, 0.0, -1.0, -2.0]], np.float32)
    g, o = run(sampler, O.QWEN, rows, uniforms=[0.5] * 3, temperature=0.001, top_k=0, top_p=1.0)
    assert g["ids"].tolist() == o["ids"].tolist() == [0, 1, 0]


@pytest.mark.parametrize("ld_pad", [0, 1, 2, 3, 5])
@pytest.mark.parametrize("V", [2, 100, 2049, 5000, 8194, 16000])
def test_qwen_shapes_and_alignment(sampler, V, ld_pad):
    g_ = np.random.default_rng(V * 10 + ld_pad)
    rows = 5
    x = (g_.standard_normal((rows, V)) * 3).astype(np.float32)
    hist = [g_.integers(0, V + 5, 40).tolist() for _ in range(rows)]  # some ids >= V
    u = [O.QwenRng(V + ld_pad).rand_f32() for _ in range(rows)]
    g, o = run(sampler, O.QWEN, x, hist, u, ld_pad=ld_pad, temperature=0.9, top_k=50, top_p=0.8, penalty=1.3)
    tie = (o["flags"] & 1) != 0
    same(g, o, rows=[r for r in range(rows) if not tie[r]])


def test_qwen_bf16(sampler):
    g_ = np.random.default_rng(5)
    V = 3000
    x = (g_.standard_normal((6, V)) * 3).astype(np.float32)
    u = [O.QwenRng(1).rand_f32() for _ in range(6)]
    for pad in (0, 1, 3):
        g, o = run(sampler, O.QWEN, x, None, u, bf16=True, ld_pad=pad, temperature=0.7, top_k=40, top_p=0.95)
        tie = (o["flags"] & 1) != 0
        same(g, o, rows=[r for r in range(6) if not tie[r]])


def test_qwen_penalty_modes_and_masks(sampler):
    g_ = np.random.default_rng(9)
    V, rows = 3072, 4
    x = (g_.standard_normal((rows, V)) * 3).astype(np.float32)
    hist = [g_.integers(0, V, 100).tolist()]
    u = [O.QwenRng(3).rand_f32() for _ in range(rows)]
    sup = O.qwen_suppression_mask(V, 2150)
    # broadcast history (apply_repetition_penalty semantics) + suppression + EOS
    g, o = run(sampler, O.QWEN, x, hist, u, hist_mode=1, add_mask=sup, eos_id=2150, temperature=0.9, top_k=50,
               top_p=0.9, penalty=1.05)
    same(g, o)
    assert all(i < 2048 for i in g["ids"])
    # mask mode (apply_repetition_penalty_with_mask)
    mask = np.zeros(V, np.float32)
    mask[g_.integers(0, V, 200)] = 1.0
    g, o = run(sampler, O.QWEN, x, None, u, hist_mode=2, pen_mask=mask, temperature=0.9, top_k=50, top_p=0.9,
               penalty=2.0)
    same(g, o)


def _talker_loop(sampler, top_k, steps=24, min_new=6):
    """The qwen talker's per-step chain (synthesis.rs:546-579, 1228-1279) with the
    penalty-mask update fused into the step: one row, the mask read and marked in
    the same launch, suppression and min-new-token EOS on."""
    g_ = np.random.default_rng(31 + top_k)
    V, eos = 3072, 2150
    sup = O.qwen_suppression_mask(V, eos)
    dsup = torch.from_numpy(sup).cuda()
    host_mask = np.zeros(V, np.float32)
    dmask = torch.zeros(V, dtype=torch.float32, device="cuda")
    rng = O.QwenRng(42)
    dho = torch.zeros(2, dtype=torch.int32, device="cuda")
    dhi = torch.zeros(1, dtype=torch.int32, device="cuda")
    got, want = [], []
    hot = g_.integers(0, 2048, 4)
    for step in range(steps):
        x = (g_.standard_normal((1, V)) * 2.5).astype(np.float32)
        x[0, hot] += 6.0  # the same few likely tokens each step, so tokens repeat
        u = np.array([rng.rand_f32()], np.float32)
        eos_id = eos if step < min_new else -1
        kw = dict(temperature=0.9, top_k=top_k, top_p=0.8, penalty=1.05, eos_id=eos_id)
        p = make_params(O.QWEN, hist_mode=2, add_mask=dsup, pen_mask=dmask, mark_mask=dmask, **kw)
        r = sampler.sample(p, torch.from_numpy(x).cuda(), dho, dhi, torch.from_numpy(u).cuda())
        torch.cuda.synchronize()
        assert r.status.cpu().item() == 0
        got.append(int(r.ids.cpu().numpy().view(np.uint32)[0]))
        op = O.make_params(O.QWEN, hist_mode=2, add_mask=sup, pen_mask=host_mask.copy(), **kw)
        o = O.sample(op, x, np.zeros(2, np.uint32), np.zeros(0, np.uint32), u, cap=CAP)
        want.append(int(o["ids"][0]))
        if want[-1] < V:
            host_mask[want[-1]] = 1.0  # synthesis.rs:572-577
    return got, want, dmask.cpu().numpy(), host_mask


@pytest.mark.parametrize("top_k", [50, 200])
def test_qwen_talker_loop_with_fused_mask_update(sampler, top_k):
    # top_k 50 runs the streaming fast path, 200 the general one
    got, want, dmask, host_mask = _talker_loop(sampler, top_k)
    assert got == want
    assert np.array_equal(dmask, host_mask)
    assert len(set(got)) < len(got)  # tokens repeat: the penalty met ids already marked


def test_mark_mask_rows_and_aliasing(sampler):
    g_ = np.random.default_rng(41)
    V, rows = 3072, 16
    x = (g_.standard_normal((rows, V)) * 3).astype(np.float32)
    u = torch.from_numpy(g_.random(rows).astype(np.float32)).cuda()
    dx = torch.from_numpy(x).cuda()
    dho = torch.zeros(rows + 1, dtype=torch.int32, device="cuda")
    dhi = torch.zeros(1, dtype=torch.int32, device="cuda")
    pm = torch.zeros(V, dtype=torch.float32, device="cuda")
    pm[g_.integers(0, V, 50)] = 1.0
    mark = pm.clone()
    p = make_params(O.QWEN, hist_mode=2, pen_mask=pm, mark_mask=mark, temperature=0.9, top_k=50,
                    top_p=0.9, penalty=1.3)
    r = sampler.sample(p, dx, dho, dhi, u)
    q = make_params(O.QWEN, hist_mode=2, pen_mask=pm, temperature=0.9, top_k=50, top_p=0.9, penalty=1.3)
    r0 = sampler.sample(q, dx, dho, dhi, u)
    torch.cuda.synchronize()
    ids = r.ids.cpu().numpy().view(np.uint32)
    assert np.array_equal(ids, r0.ids.cpu().numpy().view(np.uint32))
    want = pm.cpu().numpy()
    want[ids] = 1.0
    assert np.array_equal(mark.cpu().numpy(), want)
    # a mask marked while other rows still read it would race: refused
    bad = make_params(O.QWEN, hist_mode=2, pen_mask=pm, mark_mask=pm, temperature=0.9, top_k=50, penalty=1.3)
    with pytest.raises(_lib.TcError):
        sampler.sample(bad, dx, dho, dhi, u)


# ------------------------------------------------------------------ indextts
def test_indextts_random_rows(sampler):
    g_ = np.random.default_rng(11)
    for V in (5, 300, 8194):
        x = (g_.standard_normal((8, V)) * 4).astype(np.float32)
        x[0, :3] = x[0, 3]  # ties at the top
        hist = [g_.integers(0, V, 60).tolist() for _ in range(8)]
        u = g_.random(8)
        for k, p in ((30, 0.8), (2, 0.5), (0, 0.9), (V + 5, 0.99), (30, 1.0)):
            g, o = run(sampler, O.INDEXTTS, x, hist, u, temperature=0.8, top_k=k, top_p=p, penalty=10.0, min_keep=2)
            # more than 1024 survivors: probabilities from block sums
            same(g, o, probs_exact=not (V > KSURV and (k == 0 or k >= V)))


def test_indextts_nan_row_too_few(sampler):
    x = np.array([[0.0, np.nan, 1.0, 2.0]], np.float32)
    g, o = run(sampler, O.INDEXTTS, x, None, [0.5], temperature=0.8, top_k=30, top_p=0.8, penalty=1.0)
    assert o["status"][0] == O.ETOOFEW and g["status"][0] == _lib.TC_ETOOFEW


# ------------------------------------------------------------------ cosyvoice3
def test_cosy_ignore_eos(sampler):
    # crates/cosyvoice3/src/llm.rs:713-735
    vocab, eos = 6761, 6561
    raw = np.full((1, vocab), -20.0, np.float32)
    raw[0, eos], raw[0, 7] = 50.0, 10.0
    rng = O.StepRng(42)
    kw = dict(top_p=0.9, top_k=5, ras_win=10, ras_tau=0.1)
    g, o = run(sampler, O.COSY_RAS, raw, [[]], [rng.next_f32(), 0.0], eos_id=eos, **kw)
    assert g["ids"][0] == o["ids"][0] == 7
    g, o = run(sampler, O.COSY_RAS, raw, [[]], [rng.next_f32(), 0.0], eos_id=-1, **kw)
    assert g["ids"][0] == o["ids"][0] == eos


def test_cosy_random_rows_and_ras(sampler):
    g_ = np.random.default_rng(12)
    V = 700
    x = (g_.standard_normal((10, V)) * 3).astype(np.float32)
    x[:, 5] += 20.0
    hist = [([5] if r % 2 else [1]) + g_.integers(0, V, 5).tolist() for r in range(10)]
    u = g_.random(20).astype(np.float32)
    g, o = run(sampler, O.COSY_RAS, x, hist, u, top_p=0.8, top_k=25, ras_win=10, ras_tau=0.1)
    same(g, o)
    assert ((g["flags"] & 2) != 0).sum() >= 4


def test_cosy_fast_path_ties_eos_and_ras(sampler):
    # logits on a 0.5 grid (many equal probabilities at the top_k-th rank: the
    # reference's order is probability descending, id ascending), the
    # ignore_eos id inside the candidate range, and rows whose dominant token
    # is in the window (they draw from every probability)
    g_ = np.random.default_rng(33)
    V, rows, eos = 6564, 16, 100
    x = (np.round(g_.standard_normal((rows, V)) * 6.0) / 2.0).astype(np.float32)
    x[:, eos] = x.max(axis=1) + 1.0
    hot = g_.integers(200, V, rows)
    x[np.arange(rows), hot] = x.max(axis=1) + 6.0  # dominant: the nucleus is that one token
    hist = [(g_.integers(0, V, 7).tolist() + [int(hot[r])] * (2 if r % 2 == 0 else 0)) for r in range(rows)]
    u = g_.random(2 * rows).astype(np.float32)
    g, o = run(sampler, O.COSY_RAS, x, hist, u, top_p=0.8, top_k=25, ras_win=10, ras_tau=0.1, eos_id=eos)
    same(g, o)
    assert ((g["flags"] & 2) != 0).sum() == rows // 2
    # without the dominant token: the nucleus spans many tied ranks
    x2 = (np.round(g_.standard_normal((rows, V)) * 4.0) / 2.0).astype(np.float32)
    g, o = run(sampler, O.COSY_RAS, x2, hist, u, top_p=0.8, top_k=25, ras_win=10, ras_tau=0.1, eos_id=eos)
    same(g, o)
    assert (o["keep_count"] > 5).all()


@pytest.mark.parametrize("V,top_k,bf16", [(300, 1, False), (2048, 64, False), (6564, 25, True), (16000, 40, False),
                                          (6761, 25, False)])
def test_cosy_fast_path_shapes(sampler, V, top_k, bf16):
    # the fast path across vocabularies, top_k at both ends of its range, bf16
    # rows, the EOS id inside the row and windows that fire on every other row
    g_ = np.random.default_rng(V + top_k)
    rows = 12
    x = (g_.standard_normal((rows, V)) * 3).astype(np.float32)
    hot = g_.integers(0, V, rows)
    x[np.arange(rows), hot] = x.max(axis=1) + 5.0
    eos = int(g_.integers(0, V))
    hist = [g_.integers(0, V, 9).tolist() + ([int(hot[r])] if r % 2 else []) for r in range(rows)]
    u = g_.random(2 * rows).astype(np.float32)
    g, o = run(sampler, O.COSY_RAS, x, hist, u, bf16=bf16, ld_pad=5, top_p=0.8, top_k=top_k, ras_win=10, ras_tau=0.1,
               eos_id=eos)
    same(g, o)
    assert np.array_equal(g["flags"], o["flags"].astype(np.int32))


def test_cosy_random_picks_on_running_sums(sampler):
    # random_sample_probs (llm.rs:594-604) with the pick on the reference's f32
    # running sum at an index, one ulp either side of it, at the row's total,
    # next to 1 and at 0: draws decided at their exact boundary (tau 0: every
    # window fires); near-uniform rows put many candidates inside any error
    # window, peaked ones few
    g_ = np.random.default_rng(41)
    V, rows, eos = 6564, 36, 77
    scale = np.where(np.arange(rows) % 4 == 3, 0.05, 3.0)
    x = (g_.standard_normal((rows, V)) * scale[:, None]).astype(np.float32)
    u = np.zeros(2 * rows, np.float32)
    u[0::2] = g_.random(rows)
    below1 = np.nextafter(np.float32(1.0), np.float32(0.0))
    for r in range(rows):
        row = x[r].copy()
        row[eos] = -np.inf
        acc = np.cumsum(O.softmax(row), dtype=np.float32)  # sequential f32 adds
        a = acc[int(g_.integers(0, V))]
        pick = (a, np.nextafter(a, np.float32(0.0)), np.nextafter(a, np.float32(2.0)), acc[-1], below1,
                np.float32(0.0))[r % 6]
        u[2 * r + 1] = min(pick, below1)
    g, o = run(sampler, O.COSY_RAS, x, None, u, top_p=0.8, top_k=25, ras_win=10, ras_tau=0.0, eos_id=eos)
    same(g, o)
    assert ((g["flags"] & 2) != 0).all()


def test_qwen_fast_path_extreme_uniforms(sampler):
    # u = 0 (token 0), u = 1 (reachable: the running sum may never reach it,
    # then token 0) and u next to 1, on the fast path with and without top-p
    g_ = np.random.default_rng(77)
    V, rows = 3072, 6
    x = (g_.standard_normal((rows, V)) * 3).astype(np.float32)
    u = np.array([0.0, 1.0, np.nextafter(np.float32(1.0), np.float32(0.0)), 0.5, 1.0, 0.0], np.float32)
    for tp in (0.8, 1.0):
        g, o = run(sampler, O.QWEN, x, None, u, temperature=0.9, top_k=50, top_p=tp)
        same(g, o)


def test_cosy_invalid_params(sampler):
    x = np.zeros((1, 8), np.float32)
    with pytest.raises(_lib.TcError) as e:
        run(sampler, O.COSY_RAS, x, [[]], [0.5, 0.5], top_p=0.0, top_k=25, ras_win=10, ras_tau=0.1)
    assert e.value.code == _lib.TC_EINVAL


# ------------------------------------------------------------------ moss / nano
def test_moss_rows(sampler):
    g_ = np.random.default_rng(13)
    V = 1027
    x = (g_.standard_normal((16, V)) * 2).astype(np.float32)
    hist = [g_.integers(0, V, 30).tolist() for _ in range(16)]
    u = g_.random(16)
    for T, k, p, ex in ((0.8, 30, 0.6, -1), (1.7, 25, 0.8, 1026), (0.0, 30, 0.6, -1), (1.0, 1000, 0.99, 3)):
        g, o = run(sampler, O.MOSS, x, hist, u, temperature=T, top_k=k, top_p=p, penalty=1.1, exclude_id=ex)
        tie = (o["flags"] & 1) != 0
        same(g, o, rows=[r for r in range(16) if not tie[r]], probs_exact=False)
    bad = x[:2].copy()
    bad[0, 3] = np.nan
    bad[1, :] = NEG
    g, o = run(sampler, O.MOSS, bad, None, [0.5, 0.5], temperature=0.8, top_k=30, top_p=0.6, penalty=1.0)
    assert g["status"].tolist() == [_lib.TC_ENONFINITE] * 2


def test_nano_reference_rows(sampler):
    # crates/moss-tts/src/nano/sampling.rs:82-99
    u = [O.NanoLcg(42).next_unit()]
    x = [[0.0, 1.0, 2.0, 3.0]]
    g, _ = run(sampler, O.MOSS_NANO, x, [[]], u, temperature=1.0, top_k=4, top_p=1.0, penalty=1.0)
    assert g["ids"][0] == 2
    g, _ = run(sampler, O.MOSS_NANO, x, [[]], u, temperature=1.0, top_k=4, top_p=0.5, penalty=1.0)
    assert g["ids"][0] == 3
    g, _ = run(sampler, O.MOSS_NANO, x, [[3, 3, 3]], u, temperature=1.0, top_k=1, top_p=1.0, penalty=2.0)
    assert g["ids"][0] == 2
    g, _ = run(sampler, O.MOSS_NANO, [[np.nan]], [[]], u, temperature=1.0, top_k=1, top_p=1.0, penalty=1.0)
    assert g["status"][0] == _lib.TC_ENONFINITE
    g, _ = run(sampler, O.MOSS_NANO, [[0.0, 1.0]], [[5]], u, temperature=1.0, top_k=1, top_p=1.0, penalty=2.0)
    assert g["status"][0] == _lib.TC_EINVAL


def test_nano_rows(sampler):
    g_ = np.random.default_rng(14)
    V = 1024
    x = (g_.standard_normal((16, V)) * 2).astype(np.float32)
    hist = [g_.integers(0, V, 20).tolist() for _ in range(16)]
    lcg = O.NanoLcg(7)
    u = [lcg.next_unit() for _ in range(16)]
    for T, k, p in ((0.8, 25, 0.95), (1.0, 2, 1.0), (1.3, 1024, 0.5)):
        g, o = run(sampler, O.MOSS_NANO, x, hist, u, temperature=T, top_k=k, top_p=p, penalty=1.2)
        same(g, o, probs_exact=False)


# ------------------------------------------------------------------ building blocks
def test_building_blocks(sampler):
    L = _lib.load()
    g_ = np.random.default_rng(15)
    V, rows = 3072, 3
    x = (g_.standard_normal((rows, V)) * 3).astype(np.float32)
    ids = g_.integers(0, V + 10, 80).astype(np.uint32)
    dx = torch.from_numpy(x).cuda()
    dout = torch.empty_like(dx)
    dids = torch.from_numpy(ids.view(np.int32)).cuda()
    st = torch.cuda.current_stream().cuda_stream
    _lib.check(L.tc_apply_repetition_penalty(sampler.ctx, dx.data_ptr(), dout.data_ptr(), rows, V, V,
                                             dids.data_ptr(), ids.size, 1.05, st))
    torch.cuda.synchronize()
    assert np.array_equal(dout.cpu().numpy(), O.qwen_penalty_ids(x, ids, 1.05))
    mask = torch.zeros(V, dtype=torch.float32, device="cuda")
    _lib.check(L.tc_build_suppression_mask(mask.data_ptr(), V, 2150, st))
    torch.cuda.synchronize()
    assert np.array_equal(mask.cpu().numpy(), O.qwen_suppression_mask(V, 2150))
    _lib.check(L.tc_apply_token_suppression_with_mask(dx.data_ptr(), dout.data_ptr(), rows, V, V,
                                                      mask.data_ptr(), st))
    torch.cuda.synchronize()
    assert np.array_equal(dout.cpu().numpy(), O.qwen_add_mask(x, O.qwen_suppression_mask(V, 2150)))
    pm = torch.zeros(V, dtype=torch.float32, device="cuda")
    tok = torch.tensor([17], dtype=torch.int32, device="cuda")
    _lib.check(L.tc_update_penalty_mask(pm.data_ptr(), V, tok.data_ptr(), st))
    _lib.check(L.tc_apply_repetition_penalty_with_mask(dx.data_ptr(), dout.data_ptr(), rows, V, V,
                                                       pm.data_ptr(), 2.0, st))
    torch.cuda.synchronize()
    want = O.qwen_penalty_mask(x, pm.cpu().numpy(), 2.0)
    assert pm.cpu().numpy()[17] == 1.0 and np.array_equal(dout.cpu().numpy(), want)
    out = torch.empty(rows, dtype=torch.int32, device="cuda")
    _lib.check(L.tc_greedy_sample(dx.data_ptr(), 0, rows, V, V, out.data_ptr(), st))
    torch.cuda.synchronize()
    assert out.cpu().numpy().tolist() == [O.argmax(r) for r in x]


# ------------------------------------------------------------------ exact sequential sums
def _glibc_expf():
    import ctypes
    libm = ctypes.CDLL("libm.so.6")
    f = libm.expf
    f.restype = ctypes.c_float
    f.argtypes = [ctypes.c_float]
    return f


def _x_with_exp(expf, t):
    """A float x whose glibc expf is exactly t (searched around log t), or None."""
    x0 = np.array([np.log(np.float64(t))], np.float32).view(np.int32)[0]
    for d in range(-48, 49):
        x = np.array([x0 + d], np.int32).view(np.float32)[0]
        if expf(float(x)) == np.float32(t):
            return np.float32(x)
    return None


def _tie_row(expf, V, e, n_ties, seed):
    """Row whose running softmax sum is exactly 2^e after 2^e zero logits (terms of 1.0),
    followed by terms that are odd multiples of half the grid of binade e: each of
    those adds rounds to even, a parity only the exact sequential sum settles."""
    g = np.random.default_rng(seed)
    row = np.full(V, -40.0, np.float32)
    ones = 2 ** e
    row[:ones] = 0.0
    half = 2.0 ** (e - 24)
    p = ones
    lo_m, hi_m = int(0.025 / half) + 1, int(0.45 / half)
    tries = 0
    while n_ties and p < V - 1 and tries < 20 * n_ties + 200:
        tries += 1
        m = int(g.integers(lo_m, hi_m))
        t = (2 * m + 1) * half
        x = _x_with_exp(expf, t)
        if x is None:
            continue
        row[p] = x
        p += int(g.integers(1, 5))
        n_ties -= 1
    return row


def test_indextts_exact_sum_adversarial(sampler):
    # the log-sum must be the reference's bit for bit: sequential f32 adds of
    # glibc expf terms, then glibc logf
    expf = _glibc_expf()
    V = 4000
    g_ = np.random.default_rng(31)
    rows = [np.zeros(V, np.float32),                                   # S = V exactly
            _tie_row(expf, V, 1, 6, 1), _tie_row(expf, V, 4, 12, 2), _tie_row(expf, V, 9, 40, 3),
            np.linspace(-40.0, 0.0, V).astype(np.float32),             # sum sweeps many binades
            np.r_[np.full(1500, -100.0, np.float32), np.zeros(V - 1500, np.float32)],  # subnormal terms first
            np.r_[np.full(V - 3, -95.0, np.float32), np.float32([0.0, -1.0, -2.0])],
            (g_.standard_normal(V) * 4).astype(np.float32)]
    x = np.stack(rows)
    u = g_.random(len(rows))
    hist = [[] for _ in rows]
    for k, p in ((30, 0.8), (2, 0.5), (50, 0.95)):
        g, o = run(sampler, O.INDEXTTS, x, hist, u, temperature=0.8, top_k=k, top_p=p, penalty=1.0, min_keep=2)
        assert np.array_equal(g["norm"].view(np.uint32), o["norm"].view(np.uint32)), (g["norm"], o["norm"])
        # rows whose top-k ties leave more survivors than the LDS stage holds
        # take the register-resident path
        same(g, o, probs_exact=False)


# ------------------------------------------------------------------ qwen, large vocabulary (bf16)
@pytest.mark.parametrize("V", [16500, 50001, 151936, 262144])
def test_qwen_large_vocab_shapes(sampler, V):
    g_ = np.random.default_rng(V)
    rows = 4
    x = (g_.standard_normal((rows, V)) * 3).astype(np.float32)
    hist = [g_.integers(0, V, 300).tolist() for _ in range(rows)]
    u = g_.random(rows)
    for ld_pad, kw in ((0, dict(temperature=0.7, top_k=1000, top_p=0.95, penalty=1.1)),
                       (3, dict(temperature=1.0, top_k=50, top_p=0.8, penalty=1.05, eos_id=7)),
                       (5, dict(temperature=0.9, top_k=2000, top_p=1.0, penalty=1.0))):
        g, o = run(sampler, O.QWEN, x, hist, u, bf16=True, ld_pad=ld_pad, **kw)
        assert (g["status"] == 0).all(), g["status"]
        tie = (o["flags"] & 1) != 0
        same(g, o, rows=[r for r in range(rows) if not tie[r]])


@pytest.mark.parametrize("top_k", [1, 2, 3, 7, 64, 100, 300, 513])
def test_qwen_large_vocab_candidate_counts(sampler, top_k):
    # candidate lists from 1 to about 600 ids: the rank sort runs at every
    # power-of-two size from 2 to 1024 keys (its wave-local and block-wide
    # stages), with and without penalised ids among the candidates
    V = 151936
    g_ = np.random.default_rng(1000 + top_k)
    rows = 4
    x = (g_.standard_normal((rows, V)) * 3).astype(np.float32)
    top = np.argsort(-x, axis=1)[:, :top_k + 8]
    hist = [top[r, ::3].tolist() + g_.integers(0, V, 200).tolist() for r in range(rows)]
    u = g_.random(rows)
    for kw in (dict(temperature=0.7, top_p=0.95, penalty=1.1), dict(temperature=1.0, top_p=0.5, penalty=0.8),
               dict(temperature=0.9, top_p=1.0, penalty=1.0)):
        g, o = run(sampler, O.QWEN, x, hist, u, bf16=True, top_k=top_k, **kw)
        assert (g["status"] == 0).all(), g["status"]
        tie = (o["flags"] & 1) != 0
        same(g, o, rows=[r for r in range(rows) if not tie[r]])


def test_qwen_large_vocab_greedy_broadcast_and_unsupported(sampler):
    g_ = np.random.default_rng(5)
    V = 151936
    x = (g_.standard_normal((3, V)) * 3).astype(np.float32)
    x[1, 100:104] = x[1].max() + 1.0  # ties at the top: the first index wins
    g, o = run(sampler, O.QWEN, x, [[1, 2, 3]], [0.3, 0.6, 0.9], bf16=True, hist_mode=1, temperature=0.005,
               top_k=50, top_p=0.9, penalty=1.2)
    assert (g["status"] == 0).all()
    assert g["ids"].tolist() == o["ids"].tolist()
    assert (g["flags"] == _lib.FLAG_GREEDY).all()
    # broadcast history, sampled
    g, o = run(sampler, O.QWEN, x, [[int(v) for v in g_.integers(0, V, 500)]], [0.3, 0.6, 0.9], bf16=True,
               hist_mode=1, temperature=0.8, top_k=300, top_p=0.9, penalty=1.3)
    assert (g["status"] == 0).all()
    tie = (o["flags"] & 1) != 0
    same(g, o, rows=[r for r in range(3) if not tie[r]])
    # a NaN row: the reference's NaN top-k order is unspecified; the NaN ids
    # are left out and the row is flagged
    y = x.copy()
    y[0, 5] = np.nan
    g, _ = run(sampler, O.QWEN, y[:1], None, [0.5], bf16=True, temperature=0.8, top_k=50, top_p=0.9, penalty=1.0)
    assert g["status"][0] == 0 and g["flags"][0] & _lib.FLAG_NAN_ROW
    assert np.isfinite(y[0, g["ids"][0]]) and g["ids"][0] != 5


def _large_rows(kind, rows, V, g_):
    x = (g_.standard_normal((rows, V)) * 3).astype(np.float32)
    if kind == "spiked":       # one logit far above the rest: the K-th lies many binades below
        x[np.arange(rows), g_.integers(0, V, rows)] = np.float32(1000.0)
    elif kind == "shifted":    # N(-10, 3^2): the top values straddle zero
        x -= np.float32(10.0)
    elif kind == "max_subtracted":
        x -= x.max(axis=1, keepdims=True)
    elif kind == "peaked":     # a few huge logits, the rest a long tail
        x = np.where(g_.random((rows, V)) < 1e-4, x + 40, x).astype(np.float32)
    return x


@pytest.mark.parametrize("kind", ["spiked", "shifted", "max_subtracted", "peaked"])
def test_qwen_large_vocab_keys_far_below_the_max(sampler, kind):
    # the K-th largest key lies more than 256 bf16 keys below the largest:
    # the kernel's full 16-bit radix select
    V = 151936
    g_ = np.random.default_rng(["spiked", "shifted", "max_subtracted", "peaked"].index(kind) + 17)
    rows = 4
    x = _large_rows(kind, rows, V, g_)
    top = np.argsort(-x, axis=1)[:, :1200]
    hist = [top[r, ::7].tolist() + g_.integers(0, V, 300).tolist() for r in range(rows)]
    u = g_.random(rows)
    for kw in (dict(temperature=0.7, top_k=1000, top_p=0.95, penalty=1.1),
               dict(temperature=1.0, top_k=300, top_p=0.99, penalty=1.0),
               dict(temperature=0.9, top_k=64, top_p=1.0, penalty=2.0)):
        print(f"[large] kind={kind} {kw}", flush=True)
        g, o = run(sampler, O.QWEN, x, hist, u, bf16=True, **kw)
        assert (g["status"] == 0).all(), g["status"]
        tie = (o["flags"] & 1) != 0
        same(g, o, rows=[r for r in range(rows) if not tie[r]])


@pytest.mark.parametrize("top_k", [50, 1000])
def test_qwen_large_vocab_kth_key_distances(sampler, top_k):
    # the K-th largest bf16 key 0, 1, 127, 128, 200, 255 and 256 keys below the
    # largest (the histogram's first half, its second half, and beyond it),
    # over a N(0, 1) tail; on half the rows the largest id is in the history
    V = 151936
    g_ = np.random.default_rng(top_k)
    dists = [0, 1, 127, 128, 200, 255, 256, 129]
    rows = len(dists)
    x = g_.standard_normal((rows, V)).astype(np.float32)
    top_bits = 0x4180  # bf16 16.0
    hist = []
    for r, dk in enumerate(dists):
        ids = g_.choice(V, top_k + 20, replace=False)
        x[r, ids[0]] = np.uint32(top_bits << 16).view(np.float32)
        x[r, ids[1:top_k]] = np.uint32((top_bits - dk) << 16).view(np.float32)
        x[r, ids[top_k:]] = np.uint32((top_bits - dk - 3) << 16).view(np.float32)  # just below the K-th
        hist.append(([int(ids[0])] if r % 2 else []) + g_.integers(0, V, 100).tolist())
    u = g_.random(rows)
    for kw in (dict(temperature=0.7, top_p=0.95, penalty=1.1), dict(temperature=1.0, top_p=1.0, penalty=1.0)):
        print(f"[large] kth distances top_k={top_k} {kw}", flush=True)
        g, o = run(sampler, O.QWEN, x, hist, u, bf16=True, top_k=top_k, **kw)
        assert (g["status"] == 0).all(), g["status"]
        tie = (o["flags"] & 1) != 0
        same(g, o, rows=[r for r in range(rows) if not tie[r]])


def test_qwen_large_vocab_negative_penalty(sampler):
    # a negative penalty maps logits in reverse order (sampling.rs:388-395 does
    # not reject it): penalised ids are selected by the reversed key threshold
    V = 151936
    g_ = np.random.default_rng(77)
    rows = 4
    x = (g_.standard_normal((rows, V)) * 3).astype(np.float32)
    low = np.argsort(x, axis=1)[:, :40]     # the most negative logits become the largest
    top = np.argsort(-x, axis=1)[:, :40]
    hist = [low[r].tolist() + top[r, ::2].tolist() + g_.integers(0, V, 200).tolist() for r in range(rows)]
    u = g_.random(rows)
    for kw in (dict(temperature=0.7, top_k=50, top_p=0.9, penalty=-1.0),
               dict(temperature=1.0, top_k=1000, top_p=0.95, penalty=-2.5)):
        g, o = run(sampler, O.QWEN, x, hist, u, bf16=True, **kw)
        assert (g["status"] == 0).all(), g["status"]
        tie = (o["flags"] & 1) != 0
        same(g, o, rows=[r for r in range(rows) if not tie[r]])


def test_qwen_large_vocab_infinities(sampler):
    # +inf (after the caller chain) sends the reference's CDF to index 0;
    # -inf entries weigh zero; the EOS id forced to -inf masks a +inf there
    V = 151936
    g_ = np.random.default_rng(78)
    x = (g_.standard_normal((4, V)) * 3).astype(np.float32)
    x[0, 1234] = np.inf
    x[1, g_.integers(0, V, 5000)] = -np.inf
    x[2, 999] = np.inf     # the EOS id below: forced to -inf, so the row samples normally
    x[3, 4321] = -np.inf
    x[3, 4322] = np.inf    # penalised with a positive penalty: stays +inf
    hist = [[1], [2], [3], [4322]]
    g, o = run(sampler, O.QWEN, x, hist, g_.random(4), bf16=True, temperature=0.8, top_k=100, top_p=0.9,
               penalty=1.2, eos_id=999)
    assert (g["status"] == 0).all(), g["status"]
    assert g["ids"][0] == 0 and o["ids"][0] == 0
    assert g["ids"][3] == 0 and o["ids"][3] == 0
    tie = (o["flags"] & 1) != 0
    same(g, o, rows=[r for r in (1, 2) if not tie[r]])


def test_qwen_large_vocab_overflow(sampler):
    # finite bf16 logits that the temperature or the penalty carry past the
    # f32 range: a +inf logit sends the CDF to index 0 as a +inf input does;
    # a K-th logit of -inf keeps every id (each is >= -inf), more survivors
    # than the kernel stages, so the row reports TC_EUNSUPPORTED
    V = 151936
    g_ = np.random.default_rng(79)
    x = (g_.standard_normal((4, V)) * 3).astype(np.float32)
    x[0, 777] = np.float32(3.0e38)          # x 2 (temperature 0.5) -> +inf
    x[1, 888] = np.float32(3.0e38)          # in the history: x 1/0.6 -> +inf
    x[2, :] = np.float32(-3.0e38)           # -> -inf everywhere but 30 ids
    x[2, g_.integers(0, V, 30)] = g_.standard_normal(30).astype(np.float32)
    hist = [[1], [888], [3], [4]]
    u = g_.random(4)
    g, o = run(sampler, O.QWEN, x, hist, u, bf16=True, temperature=0.5, top_k=50, top_p=0.9, penalty=0.6)
    assert g["status"][0] == 0 and g["ids"][0] == 0 and o["ids"][0] == 0
    assert g["status"][1] == 0 and g["ids"][1] == 0 and o["ids"][1] == 0
    assert g["status"][2] == _lib.TC_EUNSUPPORTED
    assert g["status"][3] == 0
    tie = (o["flags"] & 1) != 0
    same(g, o, rows=[r for r in (3,) if not tie[r]])


@pytest.mark.parametrize("V", [16500, 151936])
def test_qwen_large_vocab_f32_rows(sampler, V):
    # f32 rows above the register-resident size: candidates selected on the
    # final logits (k_qwen_large_gen), the same finish as the bf16 kernel
    g_ = np.random.default_rng(V + 3)
    rows = 4
    x = (g_.standard_normal((rows, V)) * 3).astype(np.float32)
    x[1] -= np.float32(10.0)                              # shifted row
    x[2, g_.integers(0, V, 3)] = np.float32(40.0)         # peaked row
    hist = [g_.integers(0, V, 400).tolist() for _ in range(rows)]
    u = g_.random(rows)
    for kw in (dict(temperature=0.7, top_k=1000, top_p=0.95, penalty=1.1),
               dict(temperature=1.0, top_k=50, top_p=0.8, penalty=-1.5, eos_id=11),
               dict(temperature=0.9, top_k=7, top_p=1.0, penalty=1.0)):
        print(f"[large f32] V={V} {kw}", flush=True)
        g, o = run(sampler, O.QWEN, x, hist, u, ld_pad=1, **kw)
        assert (g["status"] == 0).all(), g["status"]
        tie = (o["flags"] & 1) != 0
        same(g, o, rows=[r for r in range(rows) if not tie[r]])


@pytest.mark.parametrize("bf16", [True, False])
def test_qwen_large_vocab_masks(sampler, bf16):
    # the talker's chain at a large vocabulary: penalty mask (TC_HIST_MASK),
    # suppression mask, EOS, temperature; and greedy over the same
    V, rows = 151936, 3
    g_ = np.random.default_rng(91 + bf16)
    x = (g_.standard_normal((rows, V)) * 3).astype(np.float32)
    eos = V - 7
    supp = np.zeros(V, np.float32)
    supp[V - 1024:] = -np.inf
    supp[eos] = 0.0
    pm = np.zeros(V, np.float32)
    pm[g_.integers(0, V, 3000)] = 1.0
    pm[np.argsort(-x[0])[:20]] = 1.0                      # penalise some of the top ids
    u = g_.random(rows)
    for kw in (dict(temperature=0.9, top_k=50, top_p=0.9, penalty=1.3, eos_id=eos),
               dict(temperature=0.7, top_k=300, top_p=0.8, penalty=0.8),
               dict(temperature=0.005, top_k=50, top_p=0.9, penalty=1.3)):
        print(f"[large masks] bf16={bf16} {kw}", flush=True)
        g, o = run(sampler, O.QWEN, x, None, u, bf16=bf16, hist_mode=2, add_mask=supp, pen_mask=pm, **kw)
        assert (g["status"] == 0).all(), g["status"]
        tie = (o["flags"] & 1) != 0
        same(g, o, rows=[r for r in range(rows) if not tie[r]])


def test_qwen_large_vocab_f32_non_finite(sampler):
    V = 151936
    g_ = np.random.default_rng(95)
    x = (g_.standard_normal((3, V)) * 3).astype(np.float32)
    x[0, 777] = np.inf                       # +inf -> index 0
    x[1, g_.integers(0, V, 4000)] = -np.inf  # -inf entries weigh zero
    x[2, 9] = np.nan                         # NaN left out, row flagged
    g, o = run(sampler, O.QWEN, x, [[1], [2], [3]], g_.random(3), temperature=0.8, top_k=100, top_p=0.9,
               penalty=1.2)
    assert (g["status"] == 0).all(), g["status"]
    assert g["ids"][0] == 0 and o["ids"][0] == 0
    tie = (o["flags"] & 1) != 0
    same(g, o, rows=[1] if not tie[1] else [])
    assert g["flags"][2] & _lib.FLAG_NAN_ROW and g["ids"][2] != 9
