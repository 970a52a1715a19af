"""Build recipe for libtalechime_hip.so (gfx950) and its generated tables.

    python -m talechime_amd.build

Steps:
  1. compile and run csrc/gen_expf_table.c (host, gcc) to produce
     csrc/_gen/expf_glibc_exc.inc and csrc/_gen/logf_glibc_exc.inc -- skipped
     when both includes are newer than the generator and tc_math.h;
  2. hipcc --offload-arch=gfx950 -c each kernel source (in parallel, one
     process per file) and -shared the objects into
     talechime_amd/libtalechime_hip.so;
  3. the same for csrc/selftest.hip into talechime_amd/libtc_selftest.so
     (on-device checks of the approximations, loaded by the tests only).

Floating-point flags are part of the contract: no contraction (the kernels
reproduce unfused reference arithmetic; explicit fma() stays fused), denormals
preserved, IEEE-correct f32 division and square root, and no packed-FP32
instructions.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(PKG, "csrc")
GEN = os.path.join(CSRC, "_gen")
ROOT = os.path.dirname(PKG)
LIB = os.path.join(PKG, "libtalechime_hip.so")
SELFTEST = os.path.join(PKG, "libtc_selftest.so")

HIPCC_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-ffp-contract=off",
    "-fno-gpu-flush-denormals-to-zero",
    "-fhip-fp32-correctly-rounded-divide-sqrt",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
]


def _newer(target: str, *deps: str) -> bool:
    if not os.path.exists(target):
        return False
    t = os.path.getmtime(target)
    return all(os.path.getmtime(d) <= t for d in deps)


def gen_tables(force: bool = False) -> None:
    os.makedirs(GEN, exist_ok=True)
    inc = os.path.join(GEN, "expf_glibc_exc.inc")
    linc = os.path.join(GEN, "logf_glibc_exc.inc")
    src = os.path.join(CSRC, "gen_expf_table.c")
    hdr = os.path.join(CSRC, "tc_math.h")
    if not force and _newer(inc, src, hdr) and _newer(linc, src, hdr):
        return
    exe = os.path.join(GEN, "gen_expf_table")
    subprocess.run(["gcc", "-O2", "-fopenmp", "-fno-fast-math", "-ffp-contract=off", "-o", exe, src, "-lm"],
                   check=True)
    subprocess.run([exe, inc + ".tmp", linc + ".tmp"], check=True)
    os.replace(inc + ".tmp", inc)
    os.replace(linc + ".tmp", linc)


def hipcc() -> str:
    for c in (shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if c and os.path.exists(c):
            return c
    raise RuntimeError("hipcc not found")


# The library's sources: the C ABI with the small kernels and the beam steps
# (sampler.hip), one file per sampler family, and the LM head.
LIB_SRCS = ["sampler.hip", "k_qwen.hip", "k_indextts.hip", "k_idx_typical.hip", "k_large.hip", "k_cosy.hip", "k_moss.hip", "lm_head.hip"]
OBJ = os.path.join(CSRC, "_gen", "obj")


def build_lib() -> str:
    os.makedirs(OBJ, exist_ok=True)
    inc = ["-I", os.path.join(ROOT, "include"), "-I", CSRC]
    jobs = []
    for name in LIB_SRCS:
        obj = os.path.join(OBJ, name.replace(".hip", ".o"))
        cmd = [hipcc(), *HIPCC_FLAGS, *inc, "-c", os.path.join(CSRC, name), "-o", obj]
        jobs.append((name, obj, subprocess.Popen(cmd)))
    failed = [name for name, _, pr in jobs if pr.wait() != 0]
    if failed:
        raise RuntimeError("hipcc failed on " + ", ".join(failed))
    out_tmp = LIB + ".tmp"
    subprocess.run([hipcc(), "--offload-arch=gfx950", "-shared", "-fPIC", *[o for _, o, _ in jobs], "-o", out_tmp],
                   check=True)
    os.replace(out_tmp, LIB)
    return LIB


def build_selftest() -> str:
    """On-device checks of the approximations (tests load it; the sampler does not)."""
    out_tmp = SELFTEST + ".tmp"
    cmd = [hipcc(), *HIPCC_FLAGS, "-shared", "-I", os.path.join(ROOT, "include"), "-I", CSRC,
           os.path.join(CSRC, "selftest.hip"), "-o", out_tmp]
    subprocess.run(cmd, check=True)
    os.replace(out_tmp, SELFTEST)
    return SELFTEST


def build(force_tables: bool = False) -> str:
    gen_tables(force_tables)
    lib = build_lib()
    build_selftest()
    return lib


if __name__ == "__main__":
    print(build(force_tables="--force" in sys.argv))
