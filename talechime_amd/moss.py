"""MOSS-TTS samplers on the device (crates/moss-tts/src/sampling.rs and
nano/sampling.rs).

    Parameters, Parameters.TEXT                    sampling.rs:6-20
    sample(logits, history, parameters, exclude, rng) -> int      sampling.rs:22
    Sampler(seed).sample(logits, history, temperature, top_k, top_p, penalty) -> int
                                                   nano/sampling.rs:4-75

moss draws one f64 uniform from rand's StdRng when it samples (not for
temperature 0, not on an error): ``rng`` here is a ``numpy.random.Generator``
(or any callable returning a float in [0, 1)); a numpy generator is rewound
when the device reports an error, so its stream advances exactly when the
reference's would.  The nano Sampler keeps the reference's 32-bit LCG and
advances it after the input checks, as the reference does.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import ClassVar

import numpy as np
import torch

from . import _lib
from ._session import as_rows, csr, sampler_for
from .sampler import make_params

__all__ = ["Parameters", "sample", "Sampler", "MossError"]


class MossError(RuntimeError):
    """The reference's anyhow errors (invalid logits, repetition token or distribution)."""


@dataclass(frozen=True)
class Parameters:
    temperature: float
    top_k: int
    top_p: float
    penalty: float
    TEXT: ClassVar["Parameters"]


Parameters.TEXT = Parameters(temperature=1.5, top_k=50, top_p=1.0, penalty=1.0)

_ERRORS = {_lib.TC_ENONFINITE: "invalid MOSS logits", _lib.TC_EINVAL: "invalid repetition token",
           _lib.TC_EDIST: "invalid sampling distribution"}


def sample(logits: torch.Tensor, history, parameters: Parameters, exclude: int | None, rng) -> int:
    x = as_rows(logits.reshape(-1))
    V = x.shape[1]
    if exclude is not None and not (0 <= exclude < V):
        raise IndexError(f"exclude id {exclude} out of range")  # values[id] panics in the reference
    draws = float(np.float32(parameters.temperature)) != 0.0
    state = rng.bit_generator.state if isinstance(rng, np.random.Generator) else None
    u = (rng.random() if isinstance(rng, np.random.Generator) else float(rng())) if draws else 0.0
    ho, hi = csr([list(history)], 1, x.device)
    s = sampler_for(x.device, 1, V)
    p = make_params(_lib.MOSS, temperature=parameters.temperature, top_k=parameters.top_k, top_p=parameters.top_p,
                    penalty=parameters.penalty, exclude_id=-1 if exclude is None else int(exclude))
    res = s.sample(p, x, ho, hi, torch.tensor([u], dtype=torch.float64, device=x.device))
    st = int(res.status[0])
    if st != _lib.TC_OK:
        if state is not None:
            rng.bit_generator.state = state
        raise MossError(_ERRORS.get(st, f"status {st}"))
    return int(res.ids.cpu().numpy().view(np.uint32)[0])


class Sampler:
    """nano/sampling.rs:4-75: one LCG per stream."""

    def __init__(self, seed: int):
        self.state = seed & 0xFFFFFFFF

    def sample(self, logits: torch.Tensor, history, temperature: float, top_k: int, top_p: float,
               penalty: float) -> int:
        x = as_rows(logits.reshape(-1))
        V = x.shape[1]
        nxt = (self.state * 1664525 + 1013904223) & 0xFFFFFFFF
        u = (nxt >> 8) / 16777216.0
        ho, hi = csr([list(history)], 1, x.device)
        s = sampler_for(x.device, 1, V)
        p = make_params(_lib.MOSS_NANO, temperature=temperature, top_k=top_k, top_p=top_p, penalty=penalty)
        res = s.sample(p, x, ho, hi, torch.tensor([u], dtype=torch.float64, device=x.device))
        st = int(res.status[0])
        if st in (_lib.TC_OK, _lib.TC_EDIST):
            self.state = nxt  # the draw happens after the input checks
        if st != _lib.TC_OK:
            raise MossError(_ERRORS.get(st, f"status {st}"))
        return int(res.ids.cpu().numpy().view(np.uint32)[0])
