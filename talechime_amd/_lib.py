"""ctypes binding of libtalechime_hip.so (the C ABI in include/talechime_hip.h).

The library must be built in-tree (``python -m talechime_amd.build``).  Loading
fails loudly when it is missing: there is no CPU fallback.  torch is imported
first so that the library resolves ``libamdhip64.so.7`` to the HIP runtime torch
already loaded (one runtime per process; device pointers stay valid across).
"""
from __future__ import annotations

import ctypes as C
import os

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libtalechime_hip.so")

TC_OK, TC_EINVAL, TC_ENONFINITE, TC_ETOOFEW, TC_EHIP, TC_ENOMEM, TC_EDIST, TC_EUNSUPPORTED = range(8)
QWEN, COSY_RAS, INDEXTTS, MOSS, MOSS_NANO = range(5)
F32, BF16 = 0, 1
HIST_PER_ROW, HIST_BROADCAST, HIST_MASK = 0, 1, 2
FLAG_TIE_CUT, FLAG_RAS, FLAG_GREEDY, FLAG_NAN_ROW, FLAG_NEAR_TIE, FLAG_EXACT_SUM = 1, 2, 4, 8, 16, 32

STATUS_NAMES = {TC_OK: "ok", TC_EINVAL: "invalid argument", TC_ENONFINITE: "non-finite logits",
                TC_ETOOFEW: "too few finite candidates", TC_EHIP: "HIP error", TC_ENOMEM: "out of memory",
                TC_EDIST: "invalid sampling distribution", TC_EUNSUPPORTED: "unsupported"}

# Symbols the header declares; the CPU test suite checks every one is exported.
EXPORTS = (
    "tc_create", "tc_destroy", "tc_sample", "tc_apply_repetition_penalty",
    "tc_apply_repetition_penalty_with_mask", "tc_build_suppression_mask",
    "tc_apply_token_suppression_with_mask", "tc_update_penalty_mask", "tc_greedy_sample",
    "tc_last_error", "tc_abi_version", "tc_indextts_beam_step", "tc_indextts_beam_step_noalloc",
    "tc_indextts_beam_search_step", "tc_lm_head", "tc_head_sample",
)


class SampleParams(C.Structure):
    _fields_ = [
        ("variant", C.c_int32),
        ("hist_mode", C.c_int32),
        ("temperature", C.c_double),
        ("top_p", C.c_double),
        ("repetition_penalty", C.c_double),
        ("top_k", C.c_uint32),
        ("min_keep", C.c_uint32),
        ("ras_win", C.c_uint32),
        ("ras_tau", C.c_float),
        ("eos_id", C.c_int32),
        ("exclude_id", C.c_int32),
        ("d_add_mask", C.c_void_p),
        ("d_pen_mask", C.c_void_p),
        ("d_mark_mask", C.c_void_p),
        ("typical", C.c_int32),
        ("typical_mass", C.c_double),
    ]


class VerifyOut(C.Structure):
    _fields_ = [
        ("cap", C.c_uint32),
        ("d_topk_count", C.c_void_p),
        ("d_topk_ids", C.c_void_p),
        ("d_keep_count", C.c_void_p),
        ("d_keep_ids", C.c_void_p),
        ("d_keep_probs", C.c_void_p),
        ("d_norm", C.c_void_p),
    ]


class TcError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"{STATUS_NAMES.get(code, code)}: {msg}")
        self.code = code


_lib = None


def load(path: str = LIB_PATH):
    """Load the library (once).  Raises if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(path):
        raise RuntimeError(f"{path} is missing: build it with `python -m talechime_amd.build` "
                           "(the sampler has no CPU fallback)")
    import torch  # noqa: F401  -- bind to torch's HIP runtime (same soname)

    L = C.CDLL(path)
    vp, sz = C.c_void_p, C.c_size_t
    L.tc_create.restype = C.c_int
    L.tc_create.argtypes = [C.c_int, sz, sz, C.POINTER(vp)]
    L.tc_destroy.restype = None
    L.tc_destroy.argtypes = [vp]
    L.tc_sample.restype = C.c_int
    L.tc_sample.argtypes = [vp, C.POINTER(SampleParams), vp, C.c_int, sz, sz, sz, vp, vp, vp, vp, vp, vp,
                            C.POINTER(VerifyOut), vp]
    L.tc_apply_repetition_penalty.restype = C.c_int
    L.tc_apply_repetition_penalty.argtypes = [vp, vp, vp, sz, sz, sz, vp, sz, C.c_double, vp]
    L.tc_apply_repetition_penalty_with_mask.restype = C.c_int
    L.tc_apply_repetition_penalty_with_mask.argtypes = [vp, vp, sz, sz, sz, vp, C.c_double, vp]
    L.tc_build_suppression_mask.restype = C.c_int
    L.tc_build_suppression_mask.argtypes = [vp, sz, C.c_uint32, vp]
    L.tc_apply_token_suppression_with_mask.restype = C.c_int
    L.tc_apply_token_suppression_with_mask.argtypes = [vp, vp, sz, sz, sz, vp, vp]
    L.tc_update_penalty_mask.restype = C.c_int
    L.tc_update_penalty_mask.argtypes = [vp, sz, vp, vp]
    L.tc_greedy_sample.restype = C.c_int
    L.tc_greedy_sample.argtypes = [vp, C.c_int, sz, sz, sz, vp, vp]
    L.tc_indextts_beam_step.restype = C.c_int
    L.tc_indextts_beam_step.argtypes = [vp, C.POINTER(SampleParams), vp, C.c_int, sz, sz, sz, sz, vp, vp, vp, vp,
                                        sz, vp, vp, vp, vp, vp]
    L.tc_lm_head.restype = C.c_int
    L.tc_lm_head.argtypes = [vp, sz, vp, C.c_int, vp, sz, sz, sz, vp, sz, vp]
    L.tc_head_sample.restype = C.c_int
    L.tc_head_sample.argtypes = [vp, C.POINTER(SampleParams), vp, sz, vp, C.c_int, vp, sz, sz, sz, vp, vp, vp, vp,
                                 vp, vp, vp, vp]
    L.tc_indextts_beam_search_step.restype = C.c_int
    L.tc_indextts_beam_search_step.argtypes = [vp, C.POINTER(SampleParams), vp, C.c_int, sz, sz, sz, sz, vp, vp,
                                               vp, sz, vp, vp, vp, vp]
    L.tc_indextts_beam_step_noalloc.restype = C.c_int
    L.tc_indextts_beam_step_noalloc.argtypes = [C.POINTER(SampleParams), vp, C.c_int, sz, sz, sz, sz, vp, vp, vp,
                                                vp, sz, vp, vp, vp, vp, vp]
    L.tc_last_error.restype = C.c_char_p
    L.tc_last_error.argtypes = []
    L.tc_abi_version.restype = C.c_int
    L.tc_abi_version.argtypes = []
    _lib = L
    return L


def check(rc: int) -> None:
    if rc != TC_OK:
        raise TcError(rc, (load().tc_last_error() or b"").decode())
