"""Host-side beam bookkeeping of the indextts beam-sample loop, consuming the
candidates of ``DeviceSampler.beam_step``.

Behaves as ``BeamHypotheses`` (early_stopping off) and ``BeamSearchScorer``
(one beam group, one returned sequence) of crates/indextts/src/generation.rs:
309-440: the same names, the same argument meaning, the same results and the
same error cases, so a caller of the device step can drive the loop of
generation.rs:619-735:

    cands = sampler.beam_step(params, logits, hist_off, hist_ids, beam_scores, nb, uniforms)
    next_scores, next_tokens, next_rows = scorer.process_step(cands, input_ids, prompt_len, V, eos)

A hypothesis is a token list of any length, which is host data, so this part
of the loop stays on the host, as the reference keeps it.
"""
from __future__ import annotations

import math

import numpy as np

__all__ = ["BeamHypotheses", "BeamSearchScorer", "BeamSearchError"]

_F64_MAX = float(np.finfo(np.float64).max)


class BeamSearchError(RuntimeError):
    """Raised where the reference's ``process`` returns an error."""


class BeamHypotheses:
    """The finished hypotheses of one batch element, at most ``num_beams`` of
    them, scored by sum of log-probs over generated_len ** length_penalty
    (generation.rs:309-362)."""

    def __init__(self, num_beams: int, length_penalty: float):
        self.num_beams = num_beams
        self.length_penalty = float(length_penalty)
        self.beams: list[tuple[float, list[int]]] = []
        self.worst_score = 1e9

    def penalized(self, sum_logprobs: float, generated_len: int) -> float:
        # a zero exponent leaves the sum as it is (no power is taken)
        if self.length_penalty == 0.0:
            return float(sum_logprobs)
        return float(sum_logprobs) / math.pow(float(generated_len), self.length_penalty)

    def add(self, hyp: list[int], sum_logprobs: float, generated_len: int) -> None:
        score = self.penalized(sum_logprobs, generated_len)
        room = len(self.beams) < self.num_beams
        if not room and not score > self.worst_score:
            return
        self.beams.append((score, list(hyp)))
        if len(self.beams) <= self.num_beams:
            self.worst_score = min(self.worst_score, score)
            return
        # over capacity: drop the first of the lowest-scored entries, then the
        # worst score is the new minimum
        drop = min(range(len(self.beams)), key=lambda i: (self.beams[i][0], i))
        del self.beams[drop]
        self.worst_score = min((b[0] for b in self.beams), default=_F64_MAX)

    def is_done(self, best_sum_logprobs: float, cur_generated_len: int) -> bool:
        """Full, and no running beam can beat the worst kept hypothesis."""
        full = len(self.beams) >= self.num_beams
        return full and self.worst_score >= self.penalized(best_sum_logprobs, cur_generated_len)


class BeamSearchScorer:
    """Per batch element: its hypotheses and whether it has finished
    (generation.rs:364-440)."""

    def __init__(self, batch: int, num_beams: int, length_penalty: float):
        self.num_beams = num_beams
        self.hyps = [BeamHypotheses(num_beams, length_penalty) for _ in range(batch)]
        self.done = [False] * batch

    def is_done(self) -> bool:
        return all(self.done)

    def process(self, batch_idx: int, candidates, input_ids, prompt_len: int, vocab: int, eos_token: int,
                pad_token: int, generated_len: int):
        """One element's step.  ``candidates``: (score, flat index beam * vocab
        + id) pairs, best first.  Walks them in order: an EOS among the first
        ``num_beams`` closes that beam's hypothesis, a later EOS is passed over,
        any other token fills the next beam slot.  Returns the slots' (scores,
        tokens, source rows); a finished element gets pad tokens."""
        nb = self.num_beams
        if self.done[batch_idx]:
            return [0.0] * nb, [pad_token] * nb, [0] * nb
        slots: list[tuple[float, int, int]] = []
        best = -math.inf
        for rank, (score, flat) in enumerate(candidates):
            if len(slots) == nb:
                break
            score, flat = float(score), int(flat)
            best = max(best, score)
            beam, token = divmod(flat, vocab)
            row = batch_idx * nb + beam
            if token != eos_token:
                slots.append((score, token, row))
            elif rank < nb:
                self.hyps[batch_idx].add(list(input_ids[row][prompt_len:]), score, generated_len)
        if len(slots) < nb:
            raise BeamSearchError(
                f"element {batch_idx}: only {len(slots)} of {nb} beam slots filled by candidates other than EOS")
        self.done[batch_idx] = self.done[batch_idx] or self.hyps[batch_idx].is_done(best, generated_len)
        return [s[0] for s in slots], [s[1] for s in slots], [s[2] for s in slots]

    def process_step(self, cands, input_ids, prompt_len: int, vocab: int, eos_token: int, generated_len: int,
                     pad_token: int | None = None):
        """Every batch element of one device beam step (generation.rs:669-699):
        ``cands`` is the ``BeamCandidates`` of ``DeviceSampler.beam_step`` (or a
        dict of numpy arrays flat/scores/status).  A non-OK element status is
        the error sample_without_replacement raises in the reference."""
        pad = eos_token if pad_token is None else pad_token
        if isinstance(cands, dict):
            flat, scores, status = (np.asarray(cands[k]) for k in ("flat", "scores", "status"))
        else:
            flat, scores, status = (getattr(cands, k).cpu().numpy() for k in ("flat", "scores", "status"))
        flat = flat.view(np.uint32)
        out_s, out_t, out_r = [], [], []
        for bi in range(flat.shape[0]):
            if status[bi] != 0:
                raise BeamSearchError(f"element {bi}: sampling failed with status {int(status[bi])}")
            cand = list(zip(scores[bi].tolist(), flat[bi].tolist()))
            s, t, r = self.process(bi, cand, input_ids, prompt_len, vocab, eos_token, pad, generated_len)
            out_s += s
            out_t += t
            out_r += r
        return out_s, out_t, out_r
