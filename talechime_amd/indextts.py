"""indextts mel-code sampling on the device (crates/indextts/src/generation.rs).

    GenerateConfig                          generation.rs:43-72 (same defaults)
    sample_rows(logits, input_ids, cfg, uniforms)
        the row processors (log_softmax, repetition penalty, the typical
        warper when cfg.typical_sampling, temperature, top-k, top-p;
        generation.rs:643-662) and one draw of
        sample_without_replacement (280-303) per row
    beam_step(logits, input_ids, beam_scores, cfg, uniforms)
        one step of the beam-sample loop (619-701): the joint scores and the
        2 * num_beams candidates of each element; with cfg.do_sample False the
        beam-search branch (671-679) instead
    BeamSearchScorer                        the host bookkeeping (309-440)

The reference draws its f64 uniforms from rand's StdRng, which is not
reproduced here: callers pass the uniforms (``rng.unit_f64`` gives the same
mapping of 64-bit outputs to [0, 1)).  ``input_ids`` are the per-row id
lists the penalty reads.
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np
import torch

from . import _lib
from ._session import as_rows, csr, sampler_for
from .beam import BeamSearchScorer
from .sampler import make_params

__all__ = ["GenerateConfig", "sample_rows", "beam_step", "BeamSearchScorer"]


@dataclass
class GenerateConfig:
    do_sample: bool = True
    top_p: float = 0.8
    top_k: int = 30
    temperature: float = 0.8
    length_penalty: float = 0.0
    num_beams: int = 3
    repetition_penalty: float = 10.0
    max_new_tokens: int = 1500
    typical_sampling: bool = False
    typical_mass: float = 0.9


def _params(cfg: GenerateConfig):
    return make_params(_lib.INDEXTTS, temperature=cfg.temperature, top_k=cfg.top_k, top_p=cfg.top_p,
                       penalty=cfg.repetition_penalty, min_keep=2, typical=cfg.typical_sampling,
                       typical_mass=cfg.typical_mass)


def _uniforms(u, n: int, dev) -> torch.Tensor:
    t = torch.as_tensor(np.asarray(u, np.float64).reshape(-1), device=dev)
    if t.numel() < n:
        raise ValueError(f"{t.numel()} uniforms for {n} draws")
    return t


def sample_rows(logits: torch.Tensor, input_ids: list, cfg: GenerateConfig, uniforms) -> torch.Tensor:
    """One token per row: the processors then one draw (n = 1).  Returns the
    ids on the device; raises on a row the reference rejects."""
    x = as_rows(logits)
    rows, V = x.shape
    ho, hi = csr(input_ids, rows, x.device)
    s = sampler_for(x.device, rows, V)
    res = s.sample(_params(cfg), x, ho, hi, _uniforms(uniforms, rows, x.device))
    st = res.status
    if bool((st != _lib.TC_OK).any()):
        raise _lib.TcError(int(st[st != _lib.TC_OK][0]), "indextts sample: a row failed on the device")
    return res.ids


def beam_step(logits: torch.Tensor, input_ids: list, beam_scores, cfg: GenerateConfig, uniforms=None):
    """The candidates of one loop step for ``batch * cfg.num_beams`` beam rows
    (beam-major per element): ``BeamCandidates`` (flat beam * V + id, joint
    score, status), ready for ``BeamSearchScorer.process_step``."""
    x = as_rows(logits)
    rows, V = x.shape
    nb = cfg.num_beams
    ho, hi = csr(input_ids, rows, x.device)
    bs = torch.as_tensor(np.asarray(beam_scores, np.float64).reshape(-1), device=x.device)
    s = sampler_for(x.device, rows, V)
    if cfg.do_sample:
        return s.beam_step(_params(cfg), x, ho, hi, bs, nb, _uniforms(uniforms, (rows // nb) * 2 * nb, x.device))
    return s.beam_search_step(_params(cfg), x, ho, hi, bs, nb)
