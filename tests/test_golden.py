"""The committed golden fixtures (tests/golden/, written by make_golden.py):
their manifest, the seeded inputs they were made from, and the oracle's
outputs on those inputs, field for field."""
import hashlib
import os

import numpy as np
import pytest

from talechime_amd import synth

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _hash(*arrays):
    h = hashlib.sha256()
    for a in arrays:
        h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()


def test_manifest():
    lines = open(os.path.join(GOLD, "MANIFEST.sha256")).read().split("\n")
    entries = [ln.split() for ln in lines if ln.strip()]
    assert len(entries) == len(synth.WORKLOADS) + 1
    for digest, fn in entries:
        assert hashlib.sha256(open(os.path.join(GOLD, fn), "rb").read()).hexdigest() == digest, fn


@pytest.mark.parametrize("name", list(synth.WORKLOADS))
def test_oracle_reproduces_fixture(oracle, name):
    w = synth.WORKLOADS[name]
    g = np.load(os.path.join(GOLD, f"{name}.npz"))
    b = synth.make_batch(w, rows=8)
    assert _hash(b.logits_f32, b.hist_off, b.hist_ids, b.uniforms) == str(g["input_sha256"])
    p = oracle.make_params(w.variant, temperature=w.temperature, top_k=w.top_k, top_p=w.top_p, penalty=w.penalty,
                           min_keep=w.min_keep, ras_win=w.ras_win, ras_tau=w.ras_tau)
    o = oracle.sample(p, b.logits_f32, b.hist_off, b.hist_ids, b.uniforms, cap=64)
    for k in ("ids", "status", "flags", "topk_count", "topk_ids", "keep_count", "keep_ids"):
        assert np.array_equal(o[k], g[k]), k
    for k in ("keep_probs", "norm"):
        assert np.array_equal(o[k].view(np.uint32), g[k].view(np.uint32)), k


def test_oracle_reproduces_beam_fixture(oracle):
    w = synth.WORKLOADS["indextts-mel-256x8194"]
    g = np.load(os.path.join(GOLD, "indextts-beam-2x3x8194.npz"))
    bb = synth.make_beam_batch(w, 2, 3)
    assert _hash(bb.logits, bb.hist_off, bb.hist_ids, bb.beam_scores, bb.uniforms) == str(g["input_sha256"])
    p = oracle.make_params(oracle.INDEXTTS, temperature=w.temperature, top_k=w.top_k, top_p=w.top_p,
                           penalty=w.penalty, min_keep=w.min_keep)
    o = oracle.idx_beam_step(p, bb.logits, bb.hist_off, bb.hist_ids, bb.beam_scores, 3, bb.uniforms, 6)
    assert np.array_equal(o["flat"], g["flat"]) and np.array_equal(o["status"], g["status"])
    assert np.array_equal(o["scores"].view(np.uint64), g["scores"].view(np.uint64))
