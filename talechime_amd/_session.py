"""Per-device sampler contexts shared by the crate mirrors (qwen, cosyvoice3,
indextts, moss): one ``DeviceSampler`` per GPU, re-created larger when a call
needs more rows or a larger vocabulary than it was made for."""
from __future__ import annotations

import threading

import torch

from .sampler import DeviceSampler

_lock = threading.Lock()
_samplers: dict[int, DeviceSampler] = {}


def sampler_for(device: torch.device, rows: int, vocab: int) -> DeviceSampler:
    idx = device.index if device.index is not None else torch.cuda.current_device()
    with _lock:
        s = _samplers.get(idx)
        if s is None or s.max_rows < rows or s.max_vocab < vocab:
            if s is not None:
                torch.cuda.synchronize(device)
                s.close()
            s = DeviceSampler(idx, max_rows=max(rows, 256), max_vocab=max(vocab, 1 << 14))
            _samplers[idx] = s
        return s


def as_rows(logits: torch.Tensor) -> torch.Tensor:
    """[V] or [B, V] logits as a 2-D GPU tensor of f32 or bf16 with unit
    stride (other float types widened to f32, as the crates' to_dtype(F32))."""
    if not logits.is_cuda:
        raise ValueError("logits must be on the GPU (the sampler has no CPU path)")
    x = logits.reshape(1, -1) if logits.dim() == 1 else logits.reshape(-1, logits.shape[-1])
    if x.dtype not in (torch.float32, torch.bfloat16):
        x = x.float()
    if x.stride(-1) != 1:
        x = x.contiguous()
    return x


def csr(histories, rows: int, device: torch.device) -> tuple[torch.Tensor, torch.Tensor]:
    """Per-row id lists as the CSR pair the C ABI reads (u32 bits in int32)."""
    import numpy as np

    if len(histories) != rows:
        raise ValueError(f"{len(histories)} histories for {rows} rows")
    lens = [len(h) for h in histories]
    off = np.zeros(rows + 1, np.uint32)
    off[1:] = np.cumsum(lens)
    ids = np.concatenate([np.asarray(h, np.uint32).reshape(-1) for h in histories]) if off[-1] else \
        np.zeros(1, np.uint32)
    return (torch.from_numpy(off.view(np.int32).copy()).to(device),
            torch.from_numpy(ids.view(np.int32).copy()).to(device))
