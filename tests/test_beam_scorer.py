"""The host-side beam bookkeeping (talechime_amd.beam) against the reference's
own tests of BeamSearchScorer (crates/indextts/src/generation.rs:917-945) and
the closed forms of BeamHypotheses (generation.rs:309-362)."""
import numpy as np
import pytest

from talechime_amd import synth
from talechime_amd.beam import BeamHypotheses, BeamSearchError, BeamSearchScorer


def test_concentrated_sampling_refills_all_beams(oracle):
    # generation.rs:917-935: two active candidates, four from the inactive beams
    scores = [0.0, -40.0, -1e9, -1e9 - 40.0, -1e9, -1e9 - 40.0]
    for us in ([0.0] * 6, [0.999999] * 6, np.linspace(0.01, 0.99, 6), [0.5, 0.2, 0.9, 0.1, 0.7, 0.3]):
        picks = oracle.idx_sample_wo_replacement(scores, 6, us)
        assert picks[:2] == [0, 1] and len(set(picks)) == 6
        cands = [(scores[i], i) for i in picks]
        scorer = BeamSearchScorer(1, 3, 0.0)
        _, tokens, _ = scorer.process(0, cands, [[7]] * 3, 1, 2, 1, 1, 1)
        assert tokens == [0, 0, 0]
        assert not scorer.is_done()


def test_undersized_candidates_do_not_signal_completion():
    # generation.rs:936-945
    scorer = BeamSearchScorer(1, 3, 0.0)
    with pytest.raises(BeamSearchError):
        scorer.process(0, [(0.0, 1)], [[7]] * 3, 1, 2, 1, 1, 1)
    assert not scorer.is_done()


def test_hypotheses_keep_the_best_num_beams():
    h = BeamHypotheses(2, 0.0)
    h.add([1], -3.0, 1)
    h.add([2], -1.0, 1)
    assert h.worst_score == -3.0 and len(h.beams) == 2
    h.add([3], -5.0, 1)  # not better than the worst: dropped
    assert sorted(b[0] for b in h.beams) == [-3.0, -1.0]
    h.add([4], -2.0, 1)  # evicts -3
    assert sorted(b[0] for b in h.beams) == [-2.0, -1.0] and h.worst_score == -2.0
    # early_stopping=False: done when the worst kept beats the best running score
    assert h.is_done(-2.5, 1) and not h.is_done(-1.5, 1)


def test_hypotheses_length_penalty():
    h = BeamHypotheses(3, 1.5)
    assert h.penalized(-8.0, 4) == -8.0 / 4.0 ** 1.5
    h.add([1, 2, 3, 4], -8.0, 4)
    assert h.beams[0][0] == -1.0 and h.worst_score == -1.0
    assert BeamHypotheses(3, 0.0).penalized(-8.0, 4) == -8.0


def test_done_element_pads_and_eos_ranks():
    scorer = BeamSearchScorer(2, 2, 0.0)
    ids = [[5, 6], [5, 7], [5, 8], [5, 9]]
    # element 0: the EOS candidate at rank 0 finishes a hypothesis; the one at
    # rank 2 (>= num_beams) is skipped; the next non-EOS fill the slots
    cands = [(-0.5, 1 * 10 + 3), (-0.6, 0 * 10 + 4), (-0.7, 0 * 10 + 3), (-0.9, 1 * 10 + 6)]
    s, t, r = scorer.process(0, cands, ids, 1, 10, 3, 0, 1)
    assert t == [4, 6] and r == [0, 1] and s == [-0.6, -0.9]
    assert scorer.hyps[0].beams == [(-0.5, [7])]
    scorer.done[1] = True
    assert scorer.process(1, cands, ids, 1, 10, 3, 0, 1) == ([0.0, 0.0], [0, 0], [0, 0])


def test_process_step_over_a_beam_step(oracle):
    # the oracle's beam step feeds the scorer: per element, num_beams slots from
    # that element's rows, tokens other than EOS, scores non-increasing
    w = synth.WORKLOADS["indextts-mel-256x8194"]
    bb = synth.make_beam_batch(w, 2, 3, first_step=False)
    p = oracle.make_params(oracle.INDEXTTS, temperature=w.temperature, top_k=w.top_k, top_p=w.top_p,
                           penalty=w.penalty, min_keep=2)
    o = oracle.idx_beam_step(p, bb.logits, bb.hist_off, bb.hist_ids, bb.beam_scores, 3, bb.uniforms, 6)
    eos = int(o["flat"][0][1] % w.vocab)  # make one drawn id the EOS token
    ids = [[1, 2, 3]] * 6
    scorer = BeamSearchScorer(2, 3, 1.0)
    s, t, r = scorer.process_step(o, ids, 1, w.vocab, eos, generated_len=2)
    assert len(t) == 6 and eos not in t
    assert all(0 <= r[i] < 3 for i in range(3)) and all(3 <= r[i] < 6 for i in range(3, 6))
    assert s[:3] == sorted(s[:3], reverse=True) and s[3:] == sorted(s[3:], reverse=True)
    bad = dict(o)
    bad["status"] = np.array([0, 3], np.int32)
    with pytest.raises(BeamSearchError):
        BeamSearchScorer(2, 3, 1.0).process_step(bad, ids, 1, w.vocab, eos, generated_len=2)
