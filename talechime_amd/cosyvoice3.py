"""cosyvoice3 speech-token sampler on the device (crates/cosyvoice3/src/llm.rs
``CosyVoice3Lm::sample`` with nucleus and repetition-aware sampling).

    sample(logits, decoded, cfg, rng, ignore_eos, *, speech_token_size) -> int

Same argument meaning as llm.rs:517: ``logits`` one row (on the GPU),
``decoded`` the tokens generated so far, ``cfg`` the ``SamplingConfig``,
``rng`` the host ``StepRng`` and ``ignore_eos`` whether the EOS id
(``speech_token_size``, the model's own field in the reference) is masked.
The RNG advances as the reference's does: one draw for the nucleus, and a
second only when the repetition window fires, so the stream stays exact; the
uniforms are peeked from a clone and committed once the device has said how
many the row used.  ``sample_rows`` does the same for several independent
streams at once (one row, one history and one StepRng each).
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np
import torch

from . import _lib
from ._session import as_rows, csr, sampler_for
from .rng import StepRng
from .sampler import make_params

__all__ = ["SamplingConfig", "StepRng", "sample", "sample_rows"]


@dataclass
class SamplingConfig:
    """crates/cosyvoice3/src/config.rs:109-133 (the same defaults)."""
    top_p: float = 0.8
    top_k: int = 25
    win_size: int = 10
    tau_r: float = 0.1
    seed: int | None = None


def sample_rows(logits: torch.Tensor, decoded: list, cfg: SamplingConfig, rngs: list, ignore_eos: bool, *,
                speech_token_size: int) -> list[int]:
    x = as_rows(logits)
    rows, V = x.shape
    if len(rngs) != rows:
        raise ValueError(f"{len(rngs)} StepRngs for {rows} rows")
    # the next two draws of every stream, from clones
    u = np.zeros(2 * rows, np.float32)
    for r, g in enumerate(rngs):
        c = g.clone()
        u[2 * r], u[2 * r + 1] = c.next_f32(), c.next_f32()
    ho, hi = csr([list(d) for d in decoded], rows, x.device)
    s = sampler_for(x.device, rows, V)
    p = make_params(_lib.COSY_RAS, top_k=cfg.top_k, top_p=cfg.top_p, ras_win=cfg.win_size, ras_tau=cfg.tau_r,
                    eos_id=speech_token_size if ignore_eos else -1)
    res = s.sample(p, x, ho, hi, torch.from_numpy(u).to(x.device))
    ids = res.ids.cpu().numpy().view(np.uint32)
    st, fl = res.status.cpu().numpy(), res.flags.cpu().numpy()
    if (st != _lib.TC_OK).any():
        raise _lib.TcError(int(st[st != _lib.TC_OK][0]), "cosyvoice3 sample: a row failed on the device")
    for r, g in enumerate(rngs):
        g.next_u32()
        if fl[r] & _lib.FLAG_RAS:
            g.next_u32()
    return [int(v) for v in ids]


def sample(logits: torch.Tensor, decoded, cfg: SamplingConfig, rng: StepRng, ignore_eos: bool, *,
           speech_token_size: int) -> int:
    """llm.rs:517-538 for one row; returns the token id."""
    return sample_rows(logits.reshape(1, -1), [decoded], cfg, [rng], ignore_eos,
                       speech_token_size=speech_token_size)[0]
