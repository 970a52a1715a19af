"""qwen3-tts sampler interface on the device (crates/qwen3-tts/src/generation/
sampling.rs, tts.rs, and the talker's caller chain in synthesis.rs).

Same names and argument meaning as the reference:

    sample(logits, config, ctx) -> [batch] token tensor   (sampling.rs:137)
    apply_repetition_penalty(logits, context_tokens, penalty)        (:334)
    apply_repetition_penalty_with_mask(logits, penalty_mask, penalty) (:368)
    greedy_sample(logits)                                           (:398)
    build_suppression_mask(vocab, eos_token_id, device)             (tts.rs:22)
    apply_token_suppression_with_mask(logits, mask)                 (tts.rs:44)
    update_penalty_mask(mask, token)                                (synthesis.rs:568)

The difference the device makes: the logits stay on the GPU and the tokens
come back as a GPU tensor (int32 holding the u32 ids); the reference copies
the logits to the host to sample (sampling.rs:148-163).  ``ctx`` is the host
``SamplingContext`` the reference owns: one uniform per row, in row order, is
drawn from it for every sampled (non-greedy) step, exactly as
multinomial_sample draws them, so seeded trajectories carry over.

``talker_step`` is the whole per-step chain of synthesis.rs:546-579 in one
launch (penalty mask, suppression mask, min-new-token EOS, the draw, and the
penalty-mask update).
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np
import torch

from . import _lib
from ._session import as_rows, sampler_for
from .rng import SamplingContext
from .sampler import make_params

__all__ = ["GenerationConfig", "SamplingContext", "sample", "apply_repetition_penalty",
           "apply_repetition_penalty_with_mask", "greedy_sample", "build_suppression_mask",
           "apply_token_suppression_with_mask", "update_penalty_mask", "talker_step"]


@dataclass
class GenerationConfig:
    """sampling.rs:96-126 (the same defaults)."""
    max_new_tokens: int = 2048
    temperature: float = 0.7
    top_k: int = 50
    top_p: float = 0.9
    repetition_penalty: float = 1.0
    eos_token_id: int | None = None
    min_new_tokens: int = 2


def _stream(dev):
    return torch.cuda.current_stream(dev).cuda_stream


def _draws(config: GenerationConfig, ctx: SamplingContext, rows: int, dev) -> torch.Tensor:
    # greedy steps (temperature < 0.01) return before multinomial_sample and
    # draw nothing (sampling.rs:187-189)
    if config.temperature < 0.01:
        return torch.zeros(rows, dtype=torch.float32, device=dev)
    return torch.from_numpy(ctx.draw(rows)).to(dev)


def _check(res) -> torch.Tensor:
    st = res.status
    if bool((st != _lib.TC_OK).any()):
        code = int(st[st != _lib.TC_OK][0])
        raise _lib.TcError(code, "qwen sample: a row failed on the device")
    return res.ids


def sample(logits: torch.Tensor, config: GenerationConfig, ctx: SamplingContext) -> torch.Tensor:
    """sampling.rs:137: temperature, greedy below 0.01, top-k, top-p, softmax
    and the inverse-CDF draw, per row.  Returns [batch] ids on the device."""
    x = as_rows(logits)
    rows, V = x.shape
    s = sampler_for(x.device, rows, V)
    p = make_params(_lib.QWEN, temperature=config.temperature, top_k=config.top_k, top_p=config.top_p)
    return _check(s.sample(p, x, None, None, _draws(config, ctx, rows, x.device)))


def apply_repetition_penalty(logits: torch.Tensor, context_tokens, penalty: float) -> torch.Tensor:
    """sampling.rs:334: every id of ``context_tokens`` (ids >= vocab ignored)
    scaled in every row, positive logits by f32(1 / penalty), others by penalty."""
    x = as_rows(logits).float().contiguous()
    rows, V = x.shape
    ids = torch.as_tensor(np.asarray(context_tokens, np.uint32).view(np.int32), device=x.device).reshape(-1)
    out = torch.empty_like(x)
    s = sampler_for(x.device, rows, V)
    _lib.check(_lib.load().tc_apply_repetition_penalty(s.ctx, x.data_ptr(), out.data_ptr(), rows, V, V,
                                                      ids.data_ptr() if ids.numel() else None, ids.numel(),
                                                      float(penalty), _stream(x.device)))
    return out.reshape(logits.shape)


def apply_repetition_penalty_with_mask(logits: torch.Tensor, penalty_mask: torch.Tensor,
                                       penalty: float) -> torch.Tensor:
    """sampling.rs:368: the same scaling where the [V] mask is > 0."""
    x = as_rows(logits).float().contiguous()
    rows, V = x.shape
    m = penalty_mask.reshape(-1).float().contiguous()
    out = torch.empty_like(x)
    _lib.check(_lib.load().tc_apply_repetition_penalty_with_mask(x.data_ptr(), out.data_ptr(), rows, V, V,
                                                                m.data_ptr(), float(penalty), _stream(x.device)))
    return out.reshape(logits.shape)


def greedy_sample(logits: torch.Tensor) -> torch.Tensor:
    """sampling.rs:398: the first index of the row maximum (NaN skipped)."""
    x = as_rows(logits)
    rows, V = x.shape
    out = torch.empty(rows, dtype=torch.int32, device=x.device)
    _lib.check(_lib.load().tc_greedy_sample(x.data_ptr(), _lib.BF16 if x.dtype == torch.bfloat16 else _lib.F32,
                                           rows, V, x.stride(0), out.data_ptr(), _stream(x.device)))
    return out


def build_suppression_mask(vocab: int, eos_token_id: int, device) -> torch.Tensor:
    """tts.rs:22: -inf for the ids in [vocab - 1024, vocab) except EOS, else 0."""
    dev = torch.device(device)
    m = torch.empty(vocab, dtype=torch.float32, device=dev)
    _lib.check(_lib.load().tc_build_suppression_mask(m.data_ptr(), vocab, int(eos_token_id), _stream(dev)))
    return m


def apply_token_suppression_with_mask(logits: torch.Tensor, mask: torch.Tensor) -> torch.Tensor:
    """tts.rs:44: logits + mask, broadcast over the rows."""
    x = as_rows(logits).float().contiguous()
    rows, V = x.shape
    m = mask.reshape(-1).float().contiguous()
    out = torch.empty_like(x)
    _lib.check(_lib.load().tc_apply_token_suppression_with_mask(x.data_ptr(), out.data_ptr(), rows, V, V,
                                                               m.data_ptr(), _stream(x.device)))
    return out.reshape(logits.shape)


def update_penalty_mask(mask: torch.Tensor, token: torch.Tensor) -> None:
    """synthesis.rs:568: mask[token] = 1 (ids >= vocab ignored), in place; the
    token is read on the device."""
    if mask.dtype != torch.float32 or not mask.is_contiguous():
        raise ValueError("the penalty mask is a contiguous f32 [V] GPU tensor")
    tok = token.reshape(-1)[:1].to(torch.int32)
    _lib.check(_lib.load().tc_update_penalty_mask(mask.data_ptr(), mask.numel(), tok.data_ptr(),
                                                 _stream(mask.device)))


def talker_step(logits: torch.Tensor, config: GenerationConfig, ctx: SamplingContext,
                penalty_mask: torch.Tensor | None, suppression_mask: torch.Tensor | None,
                token_count: int) -> torch.Tensor:
    """One talker step (synthesis.rs:546-579, 1228-1279) in one launch: the
    penalty mask (when repetition_penalty != 1), the suppression mask, EOS
    forced to -inf while token_count < min_new_tokens, the draw, then the
    sampled id marked in ``penalty_mask``.  One row; returns a [1] tensor."""
    x = as_rows(logits)
    if x.shape[0] != 1:
        raise ValueError("talker_step samples one row")
    V = x.shape[1]
    pen = config.repetition_penalty
    use_pen = abs(pen - 1.0) >= 1e-9 and penalty_mask is not None
    eos = config.eos_token_id if (config.eos_token_id is not None and token_count < config.min_new_tokens) else -1
    p = make_params(_lib.QWEN, temperature=config.temperature, top_k=config.top_k, top_p=config.top_p,
                    penalty=pen if use_pen else 1.0, eos_id=eos,
                    hist_mode=_lib.HIST_MASK if use_pen else _lib.HIST_PER_ROW,
                    add_mask=suppression_mask, pen_mask=penalty_mask if use_pen else None,
                    mark_mask=penalty_mask)
    s = sampler_for(x.device, 1, V)
    return _check(s.sample(p, x, None, None, _draws(config, ctx, 1, x.device)))
