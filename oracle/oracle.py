"""ctypes wrapper over the C restatement in ``tc_oracle.c``.

TEST INFRASTRUCTURE ONLY: this is the oracle.  It may be imported by the test
suite, by the smoke check and by the CPU-baseline leg of the benchmark, never
by the product package.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libtc_oracle.so")

QWEN, COSY_RAS, INDEXTTS, MOSS, MOSS_NANO = range(5)
HIST_PER_ROW, HIST_BROADCAST, HIST_MASK = range(3)
FLAG_TIE_CUT, FLAG_RAS, FLAG_GREEDY, FLAG_NAN_ROW = 1, 2, 4, 8
OK, EINVAL, ENONFINITE, ETOOFEW, EDIST = 0, 1, 2, 3, 6


class Params(C.Structure):
    _fields_ = [
        ("variant", C.c_int32),
        ("hist_mode", C.c_int32),
        ("temperature", C.c_double),
        ("top_p", C.c_double),
        ("penalty", C.c_double),
        ("top_k", C.c_uint32),
        ("min_keep", C.c_uint32),
        ("ras_win", C.c_uint32),
        ("ras_tau", C.c_float),
        ("eos_id", C.c_int32),
        ("exclude_id", C.c_int32),
        ("typical", C.c_int32),
        ("typical_mass", C.c_double),
        ("add_mask", C.c_void_p),
        ("pen_mask", C.c_void_p),
    ]


class Verify(C.Structure):
    _fields_ = [
        ("cap", C.c_uint32),
        ("topk_count", C.c_void_p),
        ("topk_ids", C.c_void_p),
        ("keep_count", C.c_void_p),
        ("keep_ids", C.c_void_p),
        ("keep_probs", C.c_void_p),
        ("norm", C.c_void_p),
    ]


def build() -> str:
    """Compile libtc_oracle.so in place (make)."""
    subprocess.run(["make", "-s", "-C", HERE], check=True)
    return LIB_PATH


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = C.CDLL(LIB_PATH)
        f32p, u32p, u64p = C.POINTER(C.c_float), C.POINTER(C.c_uint32), C.POINTER(C.c_uint64)
        L.tco_qwen_initial_state.restype = C.c_uint64
        L.tco_qwen_initial_state.argtypes = [C.c_uint64]
        L.tco_qwen_rand_f32.restype = C.c_float
        L.tco_qwen_rand_f32.argtypes = [u64p]
        L.tco_steprng_new.argtypes = [C.c_uint64, u64p, u64p]
        L.tco_steprng_next_u32.restype = C.c_uint32
        L.tco_steprng_next_u32.argtypes = [u64p, C.c_uint64]
        L.tco_steprng_next_f32.restype = C.c_float
        L.tco_steprng_next_f32.argtypes = [u64p, C.c_uint64]
        L.tco_nano_next_unit.restype = C.c_double
        L.tco_nano_next_unit.argtypes = [u32p]
        sz = C.c_size_t
        L.tco_qwen_penalty_ids.argtypes = [f32p, sz, sz, u32p, sz, C.c_double]
        L.tco_qwen_penalty_mask.argtypes = [f32p, sz, sz, f32p, C.c_double]
        L.tco_qwen_suppression_mask.argtypes = [f32p, sz, C.c_uint32]
        L.tco_qwen_add_mask.argtypes = [f32p, sz, sz, f32p]
        L.tco_qwen_temperature.argtypes = [f32p, sz, C.c_double]
        L.tco_qwen_top_k.argtypes = [f32p, sz, sz, u32p]
        L.tco_qwen_top_p.argtypes = [f32p, sz, C.c_double, u32p]
        L.tco_softmax_last_dim.argtypes = [f32p, sz]
        L.tco_qwen_first_cdf_index.restype = C.c_int64
        L.tco_qwen_first_cdf_index.argtypes = [f32p, sz, C.c_float]
        L.tco_argmax_f32.restype = C.c_uint32
        L.tco_argmax_f32.argtypes = [f32p, sz]
        L.tco_idx_log_softmax.argtypes = [f32p, sz]
        L.tco_idx_penalty.argtypes = [f32p, sz, u32p, sz, C.c_double]
        L.tco_idx_temperature.argtypes = [f32p, sz, C.c_double]
        L.tco_idx_top_k.argtypes = [f32p, sz, sz, sz]
        L.tco_idx_top_p.argtypes = [f32p, sz, C.c_double, sz]
        L.tco_idx_typical.argtypes = [f32p, sz, C.c_double, sz]
        L.tco_idx_inverse_cdf.restype = sz
        L.tco_idx_inverse_cdf.argtypes = [C.POINTER(C.c_double), sz, C.c_double]
        L.tco_idx_sample_wo_replacement.restype = C.c_int
        L.tco_idx_sample_wo_replacement.argtypes = [C.POINTER(C.c_double), sz, sz,
                                                    C.POINTER(C.c_double), C.POINTER(sz)]
        vp = C.c_void_p
        L.tco_idx_beam_step.restype = C.c_int
        L.tco_idx_beam_step.argtypes = [C.POINTER(Params), vp, sz, sz, sz, vp, vp, vp, vp, sz, vp, vp, vp]
        L.tco_idx_beam_search_step.restype = C.c_int
        L.tco_idx_beam_search_step.argtypes = [C.POINTER(Params), vp, sz, sz, sz, vp, vp, vp, sz, vp, vp]
        L.tco_cosy_nucleus.restype = C.c_uint32
        L.tco_cosy_nucleus.argtypes = [f32p, sz, C.c_float, sz, C.c_float, C.POINTER(C.c_int),
                                       u32p, f32p, u32p]
        L.tco_cosy_random.restype = C.c_uint32
        L.tco_cosy_random.argtypes = [f32p, sz, C.c_float]
        L.tco_sample.restype = C.c_int
        L.tco_sample.argtypes = [C.POINTER(Params), C.c_void_p, sz, sz, C.c_void_p, C.c_void_p,
                                 C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p,
                                 C.POINTER(Verify), C.c_int]
        _lib = L
    return _lib


def _fp(a):
    return a.ctypes.data_as(C.POINTER(C.c_float))


def _up(a):
    return a.ctypes.data_as(C.POINTER(C.c_uint32))


def _dp(a):
    return a.ctypes.data_as(C.POINTER(C.c_double))


# ---------------------------------------------------------------- RNGs
class QwenRng:
    """crates/qwen3-tts/src/generation/sampling.rs:18-93 (seeded mode)."""

    def __init__(self, seed: int):
        self.state = C.c_uint64(lib().tco_qwen_initial_state(seed))

    def rand_f32(self) -> np.float32:
        return np.float32(lib().tco_qwen_rand_f32(C.byref(self.state)))


class StepRng:
    """crates/cosyvoice3/src/rng.rs:150-181."""

    def __init__(self, seed: int):
        self.state, self.inc = C.c_uint64(0), C.c_uint64(0)
        lib().tco_steprng_new(seed, C.byref(self.state), C.byref(self.inc))

    def next_u32(self) -> int:
        return int(lib().tco_steprng_next_u32(C.byref(self.state), self.inc.value))

    def next_f32(self) -> np.float32:
        return np.float32(lib().tco_steprng_next_f32(C.byref(self.state), self.inc.value))


class NanoLcg:
    """crates/moss-tts/src/nano/sampling.rs:4-10,66-67."""

    def __init__(self, seed: int):
        self.state = C.c_uint32(seed & 0xFFFFFFFF)

    def next_unit(self) -> float:
        return float(lib().tco_nano_next_unit(C.byref(self.state)))


# ---------------------------------------------------------------- row functions
def qwen_penalty_ids(x, ids, penalty):
    x = np.ascontiguousarray(x, np.float32).copy()
    ids = np.ascontiguousarray(ids, np.uint32)
    rows, V = x.shape
    lib().tco_qwen_penalty_ids(_fp(x), rows, V, _up(ids), ids.size, penalty)
    return x


def qwen_penalty_mask(x, mask, penalty):
    x = np.ascontiguousarray(x, np.float32).copy()
    mask = np.ascontiguousarray(mask, np.float32)
    rows, V = x.shape
    lib().tco_qwen_penalty_mask(_fp(x), rows, V, _fp(mask), penalty)
    return x


def qwen_suppression_mask(V, eos):
    m = np.empty(V, np.float32)
    lib().tco_qwen_suppression_mask(_fp(m), V, eos)
    return m


def qwen_add_mask(x, add):
    x = np.ascontiguousarray(x, np.float32).copy()
    add = np.ascontiguousarray(add, np.float32)
    lib().tco_qwen_add_mask(_fp(x), x.shape[0], x.shape[1], _fp(add))
    return x


def qwen_top_k(row, k):
    row = np.ascontiguousarray(row, np.float32).copy()
    fl = C.c_uint32(0)
    lib().tco_qwen_top_k(_fp(row), row.size, k, C.byref(fl))
    return row, fl.value


def qwen_top_p(row, p):
    row = np.ascontiguousarray(row, np.float32).copy()
    fl = C.c_uint32(0)
    lib().tco_qwen_top_p(_fp(row), row.size, p, C.byref(fl))
    return row, fl.value


def softmax(row):
    row = np.ascontiguousarray(row, np.float32).copy()
    lib().tco_softmax_last_dim(_fp(row), row.size)
    return row


def first_cdf_index(row, thr):
    row = np.ascontiguousarray(row, np.float32)
    i = lib().tco_qwen_first_cdf_index(_fp(row), row.size, np.float32(thr))
    return None if i < 0 else int(i)


def argmax(row):
    row = np.ascontiguousarray(row, np.float32)
    return int(lib().tco_argmax_f32(_fp(row), row.size))


def idx_log_softmax(row):
    row = np.ascontiguousarray(row, np.float32).copy()
    lib().tco_idx_log_softmax(_fp(row), row.size)
    return row


def idx_penalty(row, ids, pen):
    row = np.ascontiguousarray(row, np.float32).copy()
    ids = np.ascontiguousarray(ids, np.uint32)
    lib().tco_idx_penalty(_fp(row), row.size, _up(ids), ids.size, pen)
    return row


def idx_temperature(row, t):
    row = np.ascontiguousarray(row, np.float32).copy()
    lib().tco_idx_temperature(_fp(row), row.size, t)
    return row


def idx_top_k(row, k, min_keep=2):
    row = np.ascontiguousarray(row, np.float32).copy()
    lib().tco_idx_top_k(_fp(row), row.size, k, min_keep)
    return row


def idx_top_p(row, p, min_keep=2):
    row = np.ascontiguousarray(row, np.float32).copy()
    lib().tco_idx_top_p(_fp(row), row.size, p, min_keep)
    return row


def idx_typical(row, mass, min_keep=2):
    row = np.ascontiguousarray(row, np.float32).copy()
    lib().tco_idx_typical(_fp(row), row.size, mass, min_keep)
    return row


def idx_inverse_cdf(w, u):
    w = np.ascontiguousarray(w, np.float64)
    return int(lib().tco_idx_inverse_cdf(_dp(w), w.size, u))


def idx_sample_wo_replacement(scores, n, uniforms):
    scores = np.ascontiguousarray(scores, np.float64)
    uniforms = np.ascontiguousarray(uniforms, np.float64)
    out = (C.c_size_t * max(n, 1))()
    st = lib().tco_idx_sample_wo_replacement(_dp(scores), scores.size, n, _dp(uniforms), out)
    if st != OK:
        return None
    return [int(out[i]) for i in range(n)]


def idx_beam_step(params, logits, hist_off, hist_ids, beam_scores, num_beams, uniforms, n_draws):
    """One indextts beam-sample step (generation.rs:640-701).  Returns a dict:
    flat [batch, n_draws] (beam * V + id, by score descending), scores (f64),
    status [batch]."""
    logits = np.ascontiguousarray(logits, np.float32)
    rows, V = logits.shape
    assert rows % num_beams == 0
    batch = rows // num_beams
    ho = None if hist_off is None else np.ascontiguousarray(hist_off, np.uint32)
    hi = None if hist_ids is None else np.ascontiguousarray(hist_ids, np.uint32)
    if hi is not None and hi.size == 0:
        hi = np.zeros(1, np.uint32)
    bs = np.ascontiguousarray(beam_scores, np.float64)
    un = np.ascontiguousarray(uniforms, np.float64)
    assert bs.size >= rows and un.size >= batch * n_draws
    flat = np.zeros((batch, n_draws), np.uint32)
    sc = np.zeros((batch, n_draws), np.float64)
    st = np.zeros(batch, np.int32)
    rc = lib().tco_idx_beam_step(C.byref(params), logits.ctypes.data, batch, num_beams, V,
                                 None if ho is None else ho.ctypes.data, None if hi is None else hi.ctypes.data,
                                 bs.ctypes.data, un.ctypes.data, n_draws, flat.ctypes.data, sc.ctypes.data,
                                 st.ctypes.data)
    if rc != OK:
        raise ValueError(f"tco_idx_beam_step: status {rc}")
    return {"flat": flat, "scores": sc, "status": st}


def idx_beam_search_step(params, logits, hist_off, hist_ids, beam_scores, num_beams, n_keep):
    """The do_sample = false branch (generation.rs:671-679): flat [batch, n_keep]
    and scores, the n_keep best joint scores descending."""
    logits = np.ascontiguousarray(logits, np.float32)
    rows, V = logits.shape
    assert rows % num_beams == 0
    batch = rows // num_beams
    ho = None if hist_off is None else np.ascontiguousarray(hist_off, np.uint32)
    hi = None if hist_ids is None else np.ascontiguousarray(hist_ids, np.uint32)
    if hi is not None and hi.size == 0:
        hi = np.zeros(1, np.uint32)
    bs = np.ascontiguousarray(beam_scores, np.float64)
    flat = np.zeros((batch, n_keep), np.uint32)
    sc = np.zeros((batch, n_keep), np.float64)
    rc = lib().tco_idx_beam_search_step(C.byref(params), logits.ctypes.data, batch, num_beams, V,
                                        None if ho is None else ho.ctypes.data,
                                        None if hi is None else hi.ctypes.data, bs.ctypes.data, n_keep,
                                        flat.ctypes.data, sc.ctypes.data)
    if rc != OK:
        raise ValueError(f"tco_idx_beam_search_step: status {rc}")
    return {"flat": flat, "scores": sc}


def cosy_nucleus(probs, top_p, top_k, u0):
    probs = np.ascontiguousarray(probs, np.float32)
    used = C.c_int(0)
    cap = probs.size + 1
    ids = np.zeros(cap, np.uint32)
    ps = np.zeros(cap, np.float32)
    nc = C.c_uint32(0)
    t = lib().tco_cosy_nucleus(_fp(probs), probs.size, np.float32(top_p), top_k, np.float32(u0),
                               C.byref(used), _up(ids), _fp(ps), C.byref(nc))
    return int(t), bool(used.value), ids[: nc.value].tolist()


def cosy_random(probs, u1):
    probs = np.ascontiguousarray(probs, np.float32)
    return int(lib().tco_cosy_random(_fp(probs), probs.size, np.float32(u1)))


# ---------------------------------------------------------------- batch pipeline
def make_params(variant, *, temperature=1.0, top_p=1.0, penalty=1.0, top_k=0, min_keep=2,
                ras_win=10, ras_tau=0.1, eos_id=-1, exclude_id=-1, typical=False,
                typical_mass=0.9, hist_mode=HIST_PER_ROW, add_mask=None, pen_mask=None):
    p = Params()
    p.variant, p.hist_mode = variant, hist_mode
    p.temperature, p.top_p, p.penalty = temperature, top_p, penalty
    p.top_k, p.min_keep, p.ras_win, p.ras_tau = top_k, min_keep, ras_win, ras_tau
    p.eos_id, p.exclude_id = eos_id, exclude_id
    p.typical, p.typical_mass = int(typical), typical_mass
    keep = []
    if add_mask is not None:
        a = np.ascontiguousarray(add_mask, np.float32)
        keep.append(a)
        p.add_mask = a.ctypes.data
    if pen_mask is not None:
        m = np.ascontiguousarray(pen_mask, np.float32)
        keep.append(m)
        p.pen_mask = m.ctypes.data
    p._keep = keep  # keep arrays alive with the struct
    return p


def sample(params, logits, hist_off=None, hist_ids=None, uniforms=None, *, cap=0, nthreads=1):
    """Run the full per-row pipeline.  Returns a dict of numpy arrays."""
    logits = np.ascontiguousarray(logits, np.float32)
    rows, V = logits.shape
    out = np.zeros(rows, np.uint32)
    status = np.zeros(rows, np.int32)
    flags = np.zeros(rows, np.uint32)
    ho = None if hist_off is None else np.ascontiguousarray(hist_off, np.uint32)
    hi = None if hist_ids is None else np.ascontiguousarray(hist_ids, np.uint32)
    if hi is not None and hi.size == 0:
        hi = np.zeros(1, np.uint32)
    un = np.ascontiguousarray(uniforms)
    ver = None
    res = {}
    if cap:
        res = {
            "topk_count": np.zeros(rows, np.uint32), "topk_ids": np.zeros((rows, cap), np.uint32),
            "keep_count": np.zeros(rows, np.uint32), "keep_ids": np.zeros((rows, cap), np.uint32),
            "keep_probs": np.zeros((rows, cap), np.float32), "norm": np.zeros(rows, np.float32),
        }
        ver = Verify(cap, *(res[k].ctypes.data for k in
                            ("topk_count", "topk_ids", "keep_count", "keep_ids", "keep_probs", "norm")))
    rc = lib().tco_sample(C.byref(params), logits.ctypes.data, rows, V,
                          None if ho is None else ho.ctypes.data,
                          None if hi is None else hi.ctypes.data,
                          un.ctypes.data, out.ctypes.data, status.ctypes.data, flags.ctypes.data,
                          C.byref(ver) if ver is not None else None, nthreads)
    res.update({"rc": rc, "ids": out, "status": status, "flags": flags})
    return res
