"""The allocation-free beam step (tc_indextts_beam_step_noalloc, through the C
ABI) against tc_indextts_beam_step on the same inputs: candidates, joint
scores, statuses and flags bit for bit, on two calls in a row (the second
smaller, so it runs over what the first left in the shared workspace), and
its size limit rejected on the host."""
import ctypes as C

import numpy as np
import pytest

torch = pytest.importorskip("torch")

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


def _params():
    from talechime_amd.sampler import make_params
    return make_params(_lib.INDEXTTS, temperature=W.temperature, top_k=W.top_k, top_p=W.top_p, penalty=W.penalty,
                       min_keep=2)


def _inputs(batch, batch_index, first_step):
    bb = synth.make_beam_batch(W, batch, 3, first_step=first_step, batch_index=batch_index)
    dev = torch.device("cuda", 0)
    return bb, dict(
        logits=torch.from_numpy(np.ascontiguousarray(bb.logits, np.float32)).to(dev),
        hoff=torch.from_numpy(bb.hist_off.view(np.int32).copy()).to(dev),
        hids=torch.from_numpy(bb.hist_ids.view(np.int32).copy()).to(dev),
        scores=torch.from_numpy(bb.beam_scores).to(dev),
        uni=torch.from_numpy(bb.uniforms).to(dev))


def _noalloc(t, batch, n_draws=6):
    dev = t["logits"].device
    flat = torch.full((batch, n_draws), -1, dtype=torch.int32, device=dev)
    sc = torch.full((batch, n_draws), np.nan, dtype=torch.float64, device=dev)
    st = torch.full((batch,), -1, dtype=torch.int32, device=dev)
    fl = torch.full((batch,), -1, dtype=torch.int32, device=dev)
    p = _params()
    rc = _lib.load().tc_indextts_beam_step_noalloc(
        C.byref(p), t["logits"].data_ptr(), _lib.F32, batch, 3, W.vocab, t["logits"].stride(0),
        t["hoff"].data_ptr(), t["hids"].data_ptr(), t["scores"].data_ptr(), t["uni"].data_ptr(), n_draws,
        flat.data_ptr(), sc.data_ptr(), st.data_ptr(), fl.data_ptr(), torch.cuda.current_stream(dev).cuda_stream)
    _lib.check(rc)
    torch.cuda.synchronize()
    return flat.cpu().numpy(), sc.cpu().numpy(), st.cpu().numpy(), fl.cpu().numpy()


def _with_ctx(sampler, t):
    r = sampler.beam_step(_params(), t["logits"], t["hoff"], t["hids"], t["scores"], 3, t["uni"], 6)
    torch.cuda.synchronize()
    return r.flat.cpu().numpy(), r.scores.cpu().numpy(), r.status.cpu().numpy(), r.flags.cpu().numpy()


@pytest.mark.parametrize("first_step", [False, True])
def test_noalloc_beam_step_matches_context_entry_point(sampler, first_step):
    # 85 elements x 3 beams (255 of the 256 static rows), then 20 elements
    for batch, bi in ((85, 0), (20, 1)):
        print(f"[noalloc] first_step={first_step} batch={batch} batch_index={bi}", flush=True)
        _, t = _inputs(batch, bi, first_step)
        want = _with_ctx(sampler, t)
        got = _noalloc(t, batch)
        assert (want[2] == 0).all()
        for g, w in zip(got, want):
            assert np.array_equal(g.view(np.uint8), w.view(np.uint8))


def test_noalloc_beam_step_rejects_more_rows_than_its_workspace():
    if not torch.cuda.is_available():
        pytest.skip("no GPU visible")
    _, t = _inputs(2, 0, False)
    p = _params()
    dev = t["logits"].device
    out = torch.zeros(64, dtype=torch.float64, device=dev)
    # 86 x 3 = 258 beam rows > TC_NOALLOC_BEAM_ROWS: refused before any launch
    rc = _lib.load().tc_indextts_beam_step_noalloc(
        C.byref(p), t["logits"].data_ptr(), _lib.F32, 86, 3, W.vocab, t["logits"].stride(0), t["hoff"].data_ptr(),
        t["hids"].data_ptr(), t["scores"].data_ptr(), t["uni"].data_ptr(), 6, out.data_ptr(), out.data_ptr(),
        out.data_ptr(), out.data_ptr(), torch.cuda.current_stream(dev).cuda_stream)
    assert rc == _lib.TC_EINVAL
    assert b"static workspace" in _lib.load().tc_last_error()
