"""Host-side random streams of the reference samplers.

The device kernels never draw random numbers: the caller supplies one or two
uniforms per row, drawn here from the same generators the reference crates
own, so seeded trajectories are preserved exactly.  All three generators are
pure integer arithmetic.
"""
from __future__ import annotations

import numpy as np

_M64 = (1 << 64) - 1
_PCG_MUL = 6364136223846793005
_PCG_INC = 1442695040888963407


def _xsh_rr(old: int) -> int:
    xs = (((old >> 18) ^ old) >> 27) & 0xFFFFFFFF
    rot = old >> 59
    return ((xs >> rot) | (xs << ((32 - rot) & 31))) & 0xFFFFFFFF


class SamplingContext:
    """qwen3-tts RNG and sampling state for one session.

    Mirrors ``SamplingContext`` in crates/qwen3-tts/src/generation/sampling.rs:18-93
    (seeded mode).  ``rand_f32`` returns ``(out as f32) / (u32::MAX as f32)``,
    which lies in [0, 1] (1.0 is reachable).  The reference's unseeded mode
    derives values from the wall clock and is not reproducible; here an
    unseeded context is seeded from the OS entropy source instead.
    """

    def __init__(self, seed: int | None = None):
        if seed is None:
            seed = int.from_bytes(np.random.default_rng().bytes(8), "little")
        self.reset(seed)

    def reset(self, seed: int) -> None:
        """sampling.rs:50-53: back to the initial seeded state."""
        self.state = (seed * 2685821657736338717 + _PCG_INC) & _M64
        self.seeded = True

    def next_u32(self) -> int:
        old = self.state
        self.state = (old * _PCG_MUL + _PCG_INC) & _M64
        return _xsh_rr(old)

    def rand_f32(self) -> np.float32:
        return np.float32(self.next_u32()) / np.float32(4294967295.0)

    def draw(self, n: int) -> np.ndarray:
        """``n`` consecutive uniforms, one per row in row order (sampling.rs:307-311)."""
        return np.array([self.rand_f32() for _ in range(n)], np.float32)


class StepRng:
    """cosyvoice3 PCG-XSH-RR stream (crates/cosyvoice3/src/rng.rs:150-181)."""

    def __init__(self, seed: int):
        self.state = 0
        self.inc = ((seed << 1) | 1) & _M64
        self.next_u32()
        self.state = (self.state + 0x853C49E6748FEA9D) & _M64
        self.next_u32()

    def clone(self) -> "StepRng":
        c = StepRng.__new__(StepRng)
        c.state, c.inc = self.state, self.inc
        return c

    def next_u32(self) -> int:
        old = self.state
        self.state = (old * _PCG_MUL + self.inc) & _M64
        return _xsh_rr(old)

    def next_f32(self) -> np.float32:
        return np.float32(self.next_u32() >> 8) * np.float32(1.0 / (1 << 24))


class NanoLcg:
    """MOSS-TTS-Nano LCG (crates/moss-tts/src/nano/sampling.rs:4-10,66-67)."""

    def __init__(self, seed: int):
        self.state = seed & 0xFFFFFFFF

    def next_unit(self) -> float:
        self.state = (self.state * 1664525 + 1013904223) & 0xFFFFFFFF
        return (self.state >> 8) / 16777216.0


def unit_f64(seed: int, n: int) -> np.ndarray:
    """f64 uniforms in [0, 1) as (u64 >> 11) * 2^-53 from a PCG64 stream.

    Stands in for ``rand`` 0.9's ``StdRng::random::<f64>()`` (same mapping of a
    64-bit output to [0, 1), different generator) wherever the reference draws
    f64 uniforms (indextts, moss).
    """
    return np.random.Generator(np.random.PCG64(seed)).random(n)
