"""Host-side beam bookkeeping of the indextts beam-sample loop, consuming the
candidates of ``DeviceSampler.beam_step``.

Restates crates/indextts/src/generation.rs:309-440 (``BeamHypotheses`` with
early_stopping=False, ``BeamSearchScorer`` for one beam group) with the same
names, argument meaning and errors, so a caller of the device step can run the
loop of generation.rs:619-735:

    cands = sampler.beam_step(params, logits, hist_off, hist_ids, beam_scores, nb, uniforms)
    next_scores, next_tokens, next_rows = scorer.process_step(cands, input_ids, prompt_len, V, eos)

Hypotheses hold variable-length token lists, so this stays on the host, as in
the reference.
"""
from __future__ import annotations

import math

import numpy as np

__all__ = ["BeamHypotheses", "BeamSearchScorer", "BeamSearchError"]


class BeamSearchError(RuntimeError):
    """The reference's ``candle_core::bail!`` in ``process``."""


class BeamHypotheses:
    """generation.rs:309-362."""

    def __init__(self, num_beams: int, length_penalty: float):
        self.num_beams = num_beams
        self.length_penalty = float(length_penalty)
        self.beams: list[tuple[float, list[int]]] = []
        self.worst_score = 1e9

    def penalized(self, sum_logprobs: float, generated_len: int) -> float:
        if self.length_penalty == 0.0:
            return float(sum_logprobs)  # generated_len ** 0.0 == 1.0
        return float(sum_logprobs) / math.pow(float(generated_len), self.length_penalty)

    def add(self, hyp: list[int], sum_logprobs: float, generated_len: int) -> None:
        score = self.penalized(sum_logprobs, generated_len)
        if len(self.beams) < self.num_beams or score > self.worst_score:
            self.beams.append((score, list(hyp)))
            if len(self.beams) > self.num_beams:
                lowest = 0
                for i in range(1, len(self.beams)):
                    if self.beams[i][0] < self.beams[lowest][0]:
                        lowest = i
                del self.beams[lowest]
                self.worst_score = min((b[0] for b in self.beams), default=float(np.finfo(np.float64).max))
            else:
                self.worst_score = min(self.worst_score, score)

    def is_done(self, best_sum_logprobs: float, cur_generated_len: int) -> bool:
        if len(self.beams) < self.num_beams:
            return False
        return self.worst_score >= self.penalized(best_sum_logprobs, cur_generated_len)


class BeamSearchScorer:
    """generation.rs:364-440 (num_return_sequences = 1)."""

    def __init__(self, batch: int, num_beams: int, length_penalty: float):
        self.num_beams = num_beams
        self.hyps = [BeamHypotheses(num_beams, length_penalty) for _ in range(batch)]
        self.done = [False] * batch

    def is_done(self) -> bool:
        return all(self.done)

    def process(self, batch_idx: int, candidates, input_ids, prompt_len: int, vocab: int, eos_token: int,
                pad_token: int, generated_len: int):
        """``candidates``: (score, flat index beam * vocab + id), sorted by score
        descending.  Returns per-beam-slot (scores, tokens, source rows)."""
        nb = self.num_beams
        if self.done[batch_idx]:
            return [0.0] * nb, [pad_token] * nb, [0] * nb
        next_scores, next_tokens, next_rows = [0.0] * nb, [0] * nb, [0] * nb
        beam_idx = 0
        best = -math.inf
        for rank, (score, flat) in enumerate(candidates):
            score, flat = float(score), int(flat)
            best = max(best, score)
            next_index, token = flat // vocab, flat % vocab
            if token == eos_token:
                if rank >= nb:  # only candidates in the top num_beams ranks may finish
                    continue
                row = batch_idx * nb + next_index
                self.hyps[batch_idx].add(list(input_ids[row][prompt_len:]), score, generated_len)
            else:
                next_scores[beam_idx] = score
                next_tokens[beam_idx] = token
                next_rows[beam_idx] = batch_idx * nb + next_index
                beam_idx += 1
            if beam_idx == nb:
                break
        if beam_idx < nb:
            raise BeamSearchError(f"beam search needs {nb} non-EOS candidates, got {beam_idx}")
        self.done[batch_idx] = self.done[batch_idx] or self.hyps[batch_idx].is_done(best, generated_len)
        return next_scores, next_tokens, next_rows

    def process_step(self, cands, input_ids, prompt_len: int, vocab: int, eos_token: int, generated_len: int,
                     pad_token: int | None = None):
        """Every batch element of one device beam step (generation.rs:669-699):
        ``cands`` is the ``BeamCandidates`` of ``DeviceSampler.beam_step`` (or a
        dict of numpy arrays flat/scores/status).  A non-OK element status is the
        reference's error from sample_without_replacement."""
        pad = eos_token if pad_token is None else pad_token
        get = (lambda k: np.asarray(cands[k])) if isinstance(cands, dict) else \
            (lambda k: getattr(cands, k).cpu().numpy())
        flat, scores, status = get("flat").view(np.uint32), get("scores"), get("status")
        nb = self.num_beams
        out_s, out_t, out_r = [], [], []
        for bi in range(flat.shape[0]):
            if status[bi] != 0:
                raise BeamSearchError(f"element {bi}: sampling failed with status {int(status[bi])}")
            cand = list(zip(scores[bi].tolist(), flat[bi].tolist()))
            s, t, r = self.process(bi, cand, input_ids, prompt_len, vocab, eos_token, pad, generated_len)
            out_s += s
            out_t += t
            out_r += r
        assert len(out_s) == flat.shape[0] * nb
        return out_s, out_t, out_r
