"""Batched device sampler: torch tensors in, token ids out, through the C ABI.

``DeviceSampler.sample`` is the one entry the per-crate modules
(qwen / cosyvoice3 / indextts / moss) go through.  Tensors must already be on
the GPU; nothing is copied to the host unless the caller asks for it.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass

import torch

from . import _lib
from ._lib import (BF16, COSY_RAS, F32, HIST_MASK, HIST_PER_ROW, INDEXTTS, MOSS, MOSS_NANO, QWEN,
                   SampleParams, TcError, VerifyOut, check, load)

__all__ = ["DeviceSampler", "make_params", "SampleResult", "BeamCandidates", "QWEN", "COSY_RAS", "INDEXTTS", "MOSS",
           "MOSS_NANO", "TcError"]


def make_params(variant: int, *, temperature: float = 1.0, top_p: float = 1.0, penalty: float = 1.0,
                top_k: int = 0, min_keep: int = 2, ras_win: int = 10, ras_tau: float = 0.1,
                eos_id: int = -1, exclude_id: int = -1, hist_mode: int = HIST_PER_ROW,
                add_mask: torch.Tensor | None = None, pen_mask: torch.Tensor | None = None,
                mark_mask: torch.Tensor | None = None, typical: bool = False,
                typical_mass: float = 0.9) -> SampleParams:
    """Parameters of one sampler step.  `mark_mask` ([V] f32 on the device)
    receives 1.0 at each cleanly sampled row's id, the penalty-mask update of
    synthesis.rs:568-579 fused into the step; it may be `pen_mask` itself for a
    one-row step.  `typical` / `typical_mass`: indextts's typical warper
    (GenerateConfig.typical_sampling / typical_mass)."""
    p = SampleParams()
    p.variant, p.hist_mode = variant, hist_mode
    p.temperature, p.top_p, p.repetition_penalty = float(temperature), float(top_p), float(penalty)
    p.top_k, p.min_keep, p.ras_win, p.ras_tau = int(top_k), int(min_keep), int(ras_win), float(ras_tau)
    p.eos_id, p.exclude_id = int(eos_id), int(exclude_id)
    p.typical, p.typical_mass = int(bool(typical)), float(typical_mass)
    if add_mask is not None:
        _need_cuda(add_mask, torch.float32, "add_mask")
        p.d_add_mask = add_mask.data_ptr()
    if pen_mask is not None:
        _need_cuda(pen_mask, torch.float32, "pen_mask")
        p.d_pen_mask = pen_mask.data_ptr()
    if mark_mask is not None:
        _need_cuda(mark_mask, torch.float32, "mark_mask")
        p.d_mark_mask = mark_mask.data_ptr()
    p._keep = (add_mask, pen_mask, mark_mask)  # keep the tensors alive with the struct
    return p


def _need_cuda(t: torch.Tensor, dtype, name: str) -> None:
    if not t.is_cuda:
        raise ValueError(f"{name} must be a GPU tensor")
    if dtype is not None and t.dtype != dtype:
        raise ValueError(f"{name} must be {dtype}, got {t.dtype}")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")


@dataclass
class SampleResult:
    ids: torch.Tensor            # [rows] int32 (u32 bits)
    status: torch.Tensor         # [rows] int32
    flags: torch.Tensor          # [rows] int32
    topk_count: torch.Tensor | None = None
    topk_ids: torch.Tensor | None = None
    keep_count: torch.Tensor | None = None
    keep_ids: torch.Tensor | None = None
    keep_probs: torch.Tensor | None = None
    norm: torch.Tensor | None = None


class DeviceSampler:
    """Owns one tc_ctx (the library's workspace) on one GPU."""

    def __init__(self, device: int | None = None, max_rows: int = 4096, max_vocab: int = 1 << 18):
        L = load()
        self.device = torch.cuda.current_device() if device is None else int(device)
        self._ctx = C.c_void_p()
        check(L.tc_create(self.device, max_rows, max_vocab, C.byref(self._ctx)))
        self.max_rows = max_rows
        self.max_vocab = max_vocab

    def close(self) -> None:
        if self._ctx:
            load().tc_destroy(self._ctx)
            self._ctx = C.c_void_p()

    def __del__(self):  # pragma: no cover - interpreter shutdown order
        try:
            self.close()
        except Exception:
            pass

    @property
    def ctx(self) -> C.c_void_p:
        return self._ctx

    def sample(self, params: SampleParams, logits: torch.Tensor, hist_off: torch.Tensor | None,
               hist_ids: torch.Tensor | None, uniforms: torch.Tensor, *, verify_cap: int = 0,
               stream: torch.cuda.Stream | None = None, out: SampleResult | None = None) -> SampleResult:
        if logits.dim() != 2 or logits.stride(1) != 1 or not logits.is_cuda:
            raise ValueError("logits must be a 2-D GPU tensor with unit stride in the vocab dim")
        if logits.dtype == torch.float32:
            dt = F32
        elif logits.dtype == torch.bfloat16:
            dt = BF16
        else:
            raise ValueError(f"logits dtype {logits.dtype} (f32 or bf16 expected)")
        rows, V = logits.shape
        dev = logits.device
        need_u = torch.float64 if params.variant in (INDEXTTS, MOSS, MOSS_NANO) else torch.float32
        _need_cuda(uniforms, need_u, "uniforms")
        per_row = 2 if params.variant == COSY_RAS else 1
        if uniforms.numel() < rows * per_row:
            raise ValueError("not enough uniforms")
        for m in params._keep:
            if m is not None and m.numel() < V:
                raise ValueError(f"masks need {V} entries, got {m.numel()}")
        ho = hi = None
        if hist_off is not None:
            _need_cuda(hist_off, None, "hist_off")
            _need_cuda(hist_ids, None, "hist_ids")
            if hist_off.element_size() != 4 or hist_ids.element_size() != 4:
                raise ValueError("history tensors must hold 32-bit ids")
            if params.hist_mode == HIST_PER_ROW and hist_off.numel() < rows + 1:
                raise ValueError("hist_off needs rows + 1 entries")
            ho, hi = hist_off.data_ptr(), hist_ids.data_ptr() if hist_ids.numel() else hist_off.data_ptr()
        if out is None:
            out = SampleResult(torch.empty(rows, dtype=torch.int32, device=dev),
                               torch.empty(rows, dtype=torch.int32, device=dev),
                               torch.empty(rows, dtype=torch.int32, device=dev))
        ver = None
        if verify_cap:
            out.topk_count = torch.zeros(rows, dtype=torch.int32, device=dev)
            out.topk_ids = torch.zeros(rows, verify_cap, dtype=torch.int32, device=dev)
            out.keep_count = torch.zeros(rows, dtype=torch.int32, device=dev)
            out.keep_ids = torch.zeros(rows, verify_cap, dtype=torch.int32, device=dev)
            out.keep_probs = torch.zeros(rows, verify_cap, dtype=torch.float32, device=dev)
            out.norm = torch.zeros(rows, dtype=torch.float32, device=dev)
            ver = VerifyOut(verify_cap, out.topk_count.data_ptr(), out.topk_ids.data_ptr(),
                            out.keep_count.data_ptr(), out.keep_ids.data_ptr(), out.keep_probs.data_ptr(),
                            out.norm.data_ptr())
        st = (stream or torch.cuda.current_stream(dev)).cuda_stream
        rc = load().tc_sample(self._ctx, C.byref(params), logits.data_ptr(), dt, rows, V, logits.stride(0),
                              ho, hi, uniforms.data_ptr(), out.ids.data_ptr(), out.status.data_ptr(),
                              out.flags.data_ptr(), C.byref(ver) if ver is not None else None, st)
        check(rc)
        return out


    def beam_step(self, params: SampleParams, logits: torch.Tensor, hist_off: torch.Tensor | None,
                  hist_ids: torch.Tensor | None, beam_scores: torch.Tensor, num_beams: int,
                  uniforms: torch.Tensor, n_draws: int | None = None, *,
                  stream: torch.cuda.Stream | None = None) -> BeamCandidates:
        """One indextts beam-sample step (generation.rs:640-701): the candidates
        (flat index beam * V + id, joint score) of each batch element, by score
        descending.  ``logits`` holds ``batch * num_beams`` rows, beam-major per
        element; ``n_draws`` defaults to 2 * num_beams as in the reference."""
        if params.variant != INDEXTTS:
            raise ValueError("beam_step samples indextts rows")
        if logits.dim() != 2 or logits.stride(1) != 1 or not logits.is_cuda:
            raise ValueError("logits must be a 2-D GPU tensor with unit stride in the vocab dim")
        dt = {torch.float32: F32, torch.bfloat16: BF16}.get(logits.dtype)
        if dt is None:
            raise ValueError(f"logits dtype {logits.dtype} (f32 or bf16 expected)")
        rows, V = logits.shape
        if num_beams < 1 or rows % num_beams:
            raise ValueError("rows must be a multiple of num_beams")
        batch = rows // num_beams
        n_draws = 2 * num_beams if n_draws is None else n_draws
        _need_cuda(beam_scores, torch.float64, "beam_scores")
        _need_cuda(uniforms, torch.float64, "uniforms")
        if beam_scores.numel() < rows or uniforms.numel() < batch * n_draws:
            raise ValueError("beam_scores needs one score per row and uniforms n_draws per element")
        ho = hi = None
        if hist_off is not None:
            _need_cuda(hist_off, None, "hist_off")
            _need_cuda(hist_ids, None, "hist_ids")
            if hist_off.element_size() != 4 or hist_ids.element_size() != 4 or hist_off.numel() < rows + 1:
                raise ValueError("histories: rows + 1 32-bit offsets and 32-bit ids")
            ho, hi = hist_off.data_ptr(), hist_ids.data_ptr() if hist_ids.numel() else hist_off.data_ptr()
        dev = logits.device
        out = BeamCandidates(torch.empty(batch, n_draws, dtype=torch.int32, device=dev),
                             torch.empty(batch, n_draws, dtype=torch.float64, device=dev),
                             torch.empty(batch, dtype=torch.int32, device=dev),
                             torch.empty(batch, dtype=torch.int32, device=dev))
        st = (stream or torch.cuda.current_stream(dev)).cuda_stream
        check(load().tc_indextts_beam_step(self._ctx, C.byref(params), logits.data_ptr(), dt, batch, num_beams, V,
                                           logits.stride(0), ho, hi, beam_scores.data_ptr(), uniforms.data_ptr(),
                                           n_draws, out.flat.data_ptr(), out.scores.data_ptr(),
                                           out.status.data_ptr(), out.flags.data_ptr(), st))
        return out


    def beam_search_step(self, params: SampleParams, logits: torch.Tensor, hist_off: torch.Tensor | None,
                         hist_ids: torch.Tensor | None, beam_scores: torch.Tensor, num_beams: int,
                         n_keep: int | None = None, *, stream: torch.cuda.Stream | None = None) -> BeamCandidates:
        """The beam-search branch of the same loop (do_sample = false,
        generation.rs:671-679): the n_keep best joint scores of each element
        (log_softmax and the penalty only), descending.  ``n_keep`` defaults
        to 2 * num_beams as in the reference."""
        if params.variant != INDEXTTS:
            raise ValueError("beam_search_step takes indextts rows")
        if logits.dim() != 2 or logits.stride(1) != 1 or not logits.is_cuda:
            raise ValueError("logits must be a 2-D GPU tensor with unit stride in the vocab dim")
        dt = {torch.float32: F32, torch.bfloat16: BF16}.get(logits.dtype)
        if dt is None:
            raise ValueError(f"logits dtype {logits.dtype} (f32 or bf16 expected)")
        rows, V = logits.shape
        if num_beams < 1 or rows % num_beams:
            raise ValueError("rows must be a multiple of num_beams")
        batch = rows // num_beams
        n_keep = 2 * num_beams if n_keep is None else n_keep
        _need_cuda(beam_scores, torch.float64, "beam_scores")
        if beam_scores.numel() < rows:
            raise ValueError("beam_scores needs one score per row")
        ho = hi = None
        if hist_off is not None:
            _need_cuda(hist_off, None, "hist_off")
            _need_cuda(hist_ids, None, "hist_ids")
            if hist_off.element_size() != 4 or hist_ids.element_size() != 4 or hist_off.numel() < rows + 1:
                raise ValueError("histories: rows + 1 32-bit offsets and 32-bit ids")
            ho, hi = hist_off.data_ptr(), hist_ids.data_ptr() if hist_ids.numel() else hist_off.data_ptr()
        dev = logits.device
        out = BeamCandidates(torch.empty(batch, n_keep, dtype=torch.int32, device=dev),
                             torch.empty(batch, n_keep, dtype=torch.float64, device=dev),
                             torch.empty(batch, dtype=torch.int32, device=dev),
                             torch.zeros(batch, dtype=torch.int32, device=dev))
        st = (stream or torch.cuda.current_stream(dev)).cuda_stream
        check(load().tc_indextts_beam_search_step(self._ctx, C.byref(params), logits.data_ptr(), dt, batch,
                                                  num_beams, V, logits.stride(0), ho, hi, beam_scores.data_ptr(),
                                                  n_keep, out.flat.data_ptr(), out.scores.data_ptr(),
                                                  out.status.data_ptr(), st))
        return out


    def lm_head(self, hidden: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor | None = None, *,
                out: torch.Tensor | None = None, stream: torch.cuda.Stream | None = None) -> torch.Tensor:
        """The Linear before the sampler (tc_lm_head): [rows, dim] f32 hidden
        states, [vocab, dim] f32 or bf16 weights, optional [vocab] f32 bias;
        returns [rows, vocab] f32 logits."""
        h = hidden.reshape(-1, hidden.shape[-1])
        if h.dtype != torch.float32 or h.stride(-1) != 1 or not h.is_cuda:
            raise ValueError("hidden must be f32 on the GPU with unit stride")
        if weight.dim() != 2 or not weight.is_contiguous() or not weight.is_cuda:
            raise ValueError("weight must be a contiguous [vocab, dim] GPU tensor")
        wdt = {torch.float32: F32, torch.bfloat16: BF16}.get(weight.dtype)
        if wdt is None:
            raise ValueError(f"weight dtype {weight.dtype} (f32 or bf16 expected)")
        vocab, dim = weight.shape
        if h.shape[1] != dim:
            raise ValueError("hidden and weight disagree on dim")
        if bias is not None:
            _need_cuda(bias, torch.float32, "bias")
        rows = h.shape[0]
        if out is None:
            out = torch.empty(rows, vocab, dtype=torch.float32, device=h.device)
        st = (stream or torch.cuda.current_stream(h.device)).cuda_stream
        check(load().tc_lm_head(h.data_ptr(), h.stride(0), weight.data_ptr(), wdt,
                                bias.data_ptr() if bias is not None else None, rows, dim, vocab, out.data_ptr(),
                                out.stride(0), st))
        return out

    def head_sample(self, params: SampleParams, hidden: torch.Tensor, weight: torch.Tensor,
                    bias: torch.Tensor | None, hist_off: torch.Tensor | None, hist_ids: torch.Tensor | None,
                    uniforms: torch.Tensor, *, logits: torch.Tensor | None = None,
                    stream: torch.cuda.Stream | None = None) -> SampleResult:
        """The head and the sampler in one call (tc_head_sample); ``logits``
        is the [rows, vocab] f32 buffer the head writes (allocated when None)."""
        h = hidden.reshape(-1, hidden.shape[-1])
        vocab, dim = weight.shape
        rows = h.shape[0]
        if logits is None:
            logits = torch.empty(rows, vocab, dtype=torch.float32, device=h.device)
        if h.dtype != torch.float32 or h.stride(-1) != 1 or not weight.is_contiguous():
            raise ValueError("hidden f32 with unit stride, weight contiguous")
        wdt = {torch.float32: F32, torch.bfloat16: BF16}.get(weight.dtype)
        if wdt is None:
            raise ValueError(f"weight dtype {weight.dtype} (f32 or bf16 expected)")
        need_u = torch.float64 if params.variant in (INDEXTTS, MOSS, MOSS_NANO) else torch.float32
        _need_cuda(uniforms, need_u, "uniforms")
        ho = hi = None
        if hist_off is not None:
            ho, hi = hist_off.data_ptr(), hist_ids.data_ptr() if hist_ids.numel() else hist_off.data_ptr()
        dev = h.device
        out = SampleResult(torch.empty(rows, dtype=torch.int32, device=dev),
                           torch.empty(rows, dtype=torch.int32, device=dev),
                           torch.empty(rows, dtype=torch.int32, device=dev))
        st = (stream or torch.cuda.current_stream(dev)).cuda_stream
        check(load().tc_head_sample(self._ctx, C.byref(params), h.data_ptr(), h.stride(0), weight.data_ptr(), wdt,
                                    bias.data_ptr() if bias is not None else None, rows, dim, vocab,
                                    logits.data_ptr(), ho, hi, uniforms.data_ptr(), out.ids.data_ptr(),
                                    out.status.data_ptr(), out.flags.data_ptr(), st))
        return out


@dataclass
class BeamCandidates:
    flat: torch.Tensor    # [batch, n_draws] int32 (u32 bits): beam * V + id
    scores: torch.Tensor  # [batch, n_draws] f64 joint scores, descending
    status: torch.Tensor  # [batch] int32 tc_status
    flags: torch.Tensor   # [batch] int32 tc_flag bits


def launch_shape(vocab: int, dtype: int = F32) -> tuple[int, int]:
    """(items per thread, threads per block) the library uses for one row of
    ``vocab`` logits (mirrors pick_shape in csrc/sampler.hip)."""
    pad = 7 if dtype == BF16 else 3
    for items in ((8, 16, 24) if dtype == BF16 else (8, 12, 16, 24)):
        max_t = 1024 if items <= 8 else (768 if items <= 16 else 704)
        nt = -(-(vocab + pad) // items)
        nt = max(256, -(-nt // 64) * 64)
        if nt > max_t:
            continue
        bal = -(-nt // 256) * 256
        return items, (bal if bal <= max_t else nt)
    raise ValueError(f"vocab {vocab} exceeds the register-resident kernel")
