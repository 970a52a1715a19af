"""Seeded synthetic sampler workloads.

Five workloads, one per sampler configuration the port is measured and
checked on.  Every array is a deterministic function of the workload and its
seed (a counter-based SplitMix64 stream per purpose), so the oracle and the
device see identical inputs.

  qwen-talker-1x3072      qwen semantics, 1 row x 3072 f32, history 256, pen 1.05,
                          T 0.9, top-k 50, top-p 0.8
  qwen-cp-512x2048        qwen semantics, 16 codebooks x batch 32 = 512 rows x 2048,
                          T 0.9, top-k 50, top-p 1.0, no penalty
  cosy-ras-128x6564       cosyvoice3 repetition-aware sampling, 128 rows x 6564,
                          top-k 25, top-p 0.8, window 10, tau 0.1, 2 uniforms/row
  indextts-mel-256x8194   indextts processors, 256 rows x 8194, history 1500 (Zipf 1.1),
                          pen 10, T 0.8, top-k 30, top-p 0.8, one f64 uniform/row
  qwen-stress-256x151936  qwen semantics on bf16 logits, 256 rows x 151936, history 4096,
                          pen 1.1, T 0.7, top-k 1000, top-p 0.95
"""
from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np

from . import rng as _rng

BASE_SEED = 0x7A1EC0DE

QWEN, COSY_RAS, INDEXTTS, MOSS, MOSS_NANO = range(5)

_GOLD = np.uint64(0x9E3779B97F4A7C15)


def splitmix64(x: np.ndarray) -> np.ndarray:
    """SplitMix64 finaliser, element-wise (wrapping u64 arithmetic)."""
    with np.errstate(over="ignore"):
        z = np.atleast_1d(np.asarray(x, np.uint64)) + _GOLD
        z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
        z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
        return z ^ (z >> np.uint64(31))


def stream(seed: int, purpose: int, n: int, offset: int = 0) -> np.ndarray:
    """n u64 values of the counter stream (seed, purpose)."""
    key = splitmix64(np.uint64((seed * 1000003 + purpose * 7919) & 0xFFFFFFFFFFFFFFFF))[0]
    ctr = np.arange(offset, offset + n, dtype=np.uint64)
    return splitmix64(ctr ^ key)


def unit53(u: np.ndarray) -> np.ndarray:
    return (u >> np.uint64(11)).astype(np.float64) * (1.0 / 9007199254740992.0)


def normal(seed: int, purpose: int, n: int) -> np.ndarray:
    """Box-Muller in f64 from the counter stream."""
    m = (n + 1) // 2
    u = unit53(stream(seed, purpose, 2 * m))
    r = np.sqrt(-2.0 * np.log1p(-u[:m]))
    th = 2.0 * np.pi * u[m:]
    z = np.empty(2 * m)
    z[0::2] = r * np.cos(th)
    z[1::2] = r * np.sin(th)
    return z[:n]


def to_bf16_bits(x32: np.ndarray) -> np.ndarray:
    """f32 -> bf16 bit patterns, round to nearest even (finite inputs)."""
    b = x32.astype(np.float32).view(np.uint32)
    rnd = ((b >> 16) & 1) + 0x7FFF
    return ((b + rnd) >> 16).astype(np.uint16)


def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    return (b.astype(np.uint32) << 16).view(np.float32)


def uniform_ids(seed: int, purpose: int, n: int, V: int) -> np.ndarray:
    """Uniform ids in [0, V) by rejection (no modulo bias)."""
    out = np.empty(0, np.uint32)
    limit = (1 << 32) // V * V
    off = 0
    while out.size < n:
        want = (n - out.size) * 2 + 64
        u = (stream(seed, purpose, want, off) >> np.uint64(32)).astype(np.uint64)
        off += want
        u = u[u < limit]
        out = np.concatenate([out, (u % np.uint64(V)).astype(np.uint32)])
    return out[:n]


def zipf_ids(seed: int, purpose: int, n: int, V: int, s: float) -> np.ndarray:
    """Zipf(s) over ranks 1..V by an f64 inverse-CDF table; rank -> id fixed by the seed."""
    w = np.arange(1, V + 1, dtype=np.float64) ** (-s)
    cdf = np.cumsum(w)
    cdf /= cdf[-1]
    u = unit53(stream(seed, purpose, n))
    rank = np.minimum(np.searchsorted(cdf, u, side="right"), V - 1)
    perm = np.argsort(stream(seed, purpose + 1, V), kind="stable").astype(np.uint32)
    return perm[rank]


@dataclass
class Workload:
    name: str
    variant: int
    rows: int
    vocab: int
    dtype: str                 # "f32" | "bf16"
    sigma: float
    temperature: float
    top_k: int
    top_p: float
    penalty: float
    hist_len: int              # ids per row (0 = none)
    hist_kind: str             # "uniform" | "zipf" | "none"
    n_uniforms: int
    uniform_kind: str          # "qwen" | "steprng" | "f64"
    seed_index: int
    ras_win: int = 10
    ras_tau: float = 0.1
    min_keep: int = 2
    extra: dict = field(default_factory=dict)

    @property
    def seed(self) -> int:
        return BASE_SEED + self.seed_index

    @property
    def logit_bytes(self) -> int:
        return 2 if self.dtype == "bf16" else 4

    def hist_used(self) -> int:
        """History ids the kernel reads per row (the RAS window for cosyvoice3)."""
        if self.variant == COSY_RAS:
            return min(self.ras_win, self.hist_len)
        return self.hist_len

    def algorithmic_bytes_per_row(self) -> int:
        ub = 8 if self.uniform_kind == "f64" else 4
        return self.vocab * self.logit_bytes + self.hist_used() * 4 + self.n_uniforms * ub + 4


WORKLOADS = {
    "qwen-talker-1x3072": Workload("qwen-talker-1x3072", QWEN, 1, 3072, "f32", 3.0, 0.9, 50, 0.8,
                                   1.05, 256, "uniform", 1, "qwen", 0),
    "qwen-cp-512x2048": Workload("qwen-cp-512x2048", QWEN, 512, 2048, "f32", 2.5, 0.9, 50, 1.0,
                                 1.0, 0, "none", 1, "qwen", 1),
    "cosy-ras-128x6564": Workload("cosy-ras-128x6564", COSY_RAS, 128, 6564, "f32", 3.0, 1.0, 25, 0.8,
                                  1.0, 512, "uniform", 2, "steprng", 2),
    "indextts-mel-256x8194": Workload("indextts-mel-256x8194", INDEXTTS, 256, 8194, "f32", 4.0, 0.8,
                                      30, 0.8, 10.0, 1500, "zipf", 1, "f64", 3),
    "qwen-stress-256x151936": Workload("qwen-stress-256x151936", QWEN, 256, 151936, "bf16", 3.0, 0.7,
                                       1000, 0.95, 1.1, 4096, "uniform", 1, "qwen", 4),
}


@dataclass
class Batch:
    logits: np.ndarray          # [rows, V] f32 or uint16 (bf16 bits)
    logits_f32: np.ndarray      # [rows, V] f32 (exact upcast)
    hist_off: np.ndarray        # [rows + 1] u32 CSR offsets
    hist_ids: np.ndarray        # [nnz] u32
    uniforms: np.ndarray        # [rows * n_uniforms] f32 or f64


def make_batch(w: Workload, rows: int | None = None, batch_index: int = 0) -> Batch:
    """The seeded batch for workload ``w`` (first ``rows`` rows, default all)."""
    R = w.rows if rows is None else rows
    V = w.vocab
    seed = w.seed + 7777 * batch_index
    z = normal(seed, 1, R * V).reshape(R, V) * w.sigma
    x32 = z.astype(np.float32)
    if w.variant == COSY_RAS:
        # 4 rows in every 128 carry one spiked id (+12)
        spike_rows = [r for r in range(R) if r % 32 == 7]
        spike_ids = uniform_ids(seed, 5, max(len(spike_rows), 1), V)
        for j, r in enumerate(spike_rows):
            x32[r, spike_ids[j]] += np.float32(12.0)
    if w.dtype == "bf16":
        bits = to_bf16_bits(x32)
        logits, logits_f32 = bits, bf16_bits_to_f32(bits)
    else:
        logits, logits_f32 = x32, x32
    H = w.hist_len
    if H and w.hist_kind != "none":
        if w.hist_kind == "zipf":
            ids = zipf_ids(seed, 3, R * H, V, 1.1)
        else:
            ids = uniform_ids(seed, 3, R * H, V)
        ids = ids.reshape(R, H).copy()
        if w.variant == COSY_RAS:
            for j, r in enumerate(r for r in range(R) if r % 32 == 7):
                if j % 2 == 0:
                    ids[r, H - 3] = spike_ids[j]
        hist_ids = ids.reshape(-1).astype(np.uint32)
        hist_off = (np.arange(R + 1, dtype=np.uint64) * H).astype(np.uint32)
    else:
        hist_ids = np.zeros(0, np.uint32)
        hist_off = np.zeros(R + 1, np.uint32)
    if w.uniform_kind == "qwen":
        uniforms = _rng.SamplingContext(seed).draw(R)
    elif w.uniform_kind == "steprng":
        r_ = _rng.StepRng(seed)
        uniforms = np.array([r_.next_f32() for _ in range(R * w.n_uniforms)], np.float32)
    else:
        uniforms = _rng.unit_f64(seed, R * w.n_uniforms)
    return Batch(logits, logits_f32, hist_off, hist_ids, uniforms)


@dataclass
class BeamBatch:
    logits: np.ndarray       # [batch * num_beams, V] f32; row bi * num_beams + j is beam j
    hist_off: np.ndarray     # [rows + 1] u32
    hist_ids: np.ndarray     # u32
    beam_scores: np.ndarray  # [rows] f64 running beam scores
    uniforms: np.ndarray     # [batch * n_draws] f64
    num_beams: int
    n_draws: int


def make_beam_batch(w: Workload, batch: int, num_beams: int = 3, first_step: bool = False,
                    batch_index: int = 0) -> BeamBatch:
    """Inputs of one indextts beam-sample step over the seeded rows of ``w``:
    ``batch`` elements of ``num_beams`` rows each, 2 * num_beams draws per
    element (generation.rs:620).  The first step's beam scores are 0 for beam 0
    and -1e9 for the others (generation.rs:582-585); later steps carry running
    sums of log-probabilities."""
    rows = batch * num_beams
    b = make_batch(w, rows=rows, batch_index=batch_index)
    seed = w.seed + 7777 * batch_index + 0xB3A
    if first_step:
        bonus = np.array([0.0 if r % num_beams == 0 else -1e9 for r in range(rows)])
    else:
        bonus = -_rng.unit_f64(seed, rows) * 40.0
    n_draws = 2 * num_beams
    return BeamBatch(b.logits_f32, b.hist_off, b.hist_ids, bonus, _rng.unit_f64(seed + 1, batch * n_draws),
                     num_beams, n_draws)
