"""The host random streams (talechime_amd/rng.py) pinned to published values.

The device never draws random numbers: callers draw uniforms on the host from
these mirrors of the reference generators, so they carry the seeded
trajectories and must match the reference bit for bit.
"""
import numpy as np

from talechime_amd import rng

M64 = (1 << 64) - 1


def test_sampling_context_seed42_outputs():
    # crates/qwen3-tts/src/generation/sampling.rs:75-93: seed 42 gives these
    # XSH-RR outputs of the old state (integers, so exact)
    c = rng.SamplingContext(42)
    assert [c.next_u32() for _ in range(3)] == [213896069, 1518578345, 893660385]


def test_sampling_context_rand_f32_mapping_and_reset():
    # rand_f32 = (out as f32) / (u32::MAX as f32): round the integer to f32 first
    c = rng.SamplingContext(42)
    want = [np.float32(o) / np.float32(4294967295.0) for o in (213896069, 1518578345, 893660385)]
    got = [c.rand_f32() for _ in range(3)]
    assert [g.view(np.uint32) for g in got] == [w.view(np.uint32) for w in want]
    # reset returns to the seeded state (sampling.rs:50-53)
    c.reset(42)
    assert c.next_u32() == 213896069
    # one uniform per row in row order (sampling.rs:307-311)
    c.reset(42)
    d = c.draw(3)
    assert d.dtype == np.float32 and list(d) == want
    # the map reaches 1.0 exactly: outputs >= 2^32 - 128 round to 2^32 as f32
    assert np.float32(4294967295) / np.float32(4294967295.0) == np.float32(1.0)
    assert np.float32(4294967168) / np.float32(4294967295.0) == np.float32(1.0)


def test_step_rng_core_matches_pcg32_published_vector():
    # StepRng (crates/cosyvoice3/src/rng.rs:150-181) is PCG-XSH-RR 64/32 with
    # pcg32_srandom seeding (state 0, step, add initstate, step).  The PCG
    # paper's reference demo seeds initstate 42, initseq 54 and prints
    # 0xa15c02b7 0x7b47f409 0xba1d3330 0x83d2f293 0xbfa4784b 0xcbed606e.
    r = rng.StepRng.__new__(rng.StepRng)
    r.inc = ((54 << 1) | 1) & M64
    r.state = 0
    r.next_u32()
    r.state = (r.state + 42) & M64
    r.next_u32()
    assert [r.next_u32() for _ in range(6)] == [0xA15C02B7, 0x7B47F409, 0xBA1D3330, 0x83D2F293,
                                                 0xBFA4784B, 0xCBED606E]


def test_step_rng_seeding_is_srandom_with_fixed_initstate():
    # StepRng::new(seed) = pcg32_srandom(0x853C49E6748FEA9D, seed)
    for seed in (0, 7, 42, 2**63 + 5):
        a = rng.StepRng(seed)
        b = rng.StepRng.__new__(rng.StepRng)
        b.inc = ((seed << 1) | 1) & M64
        b.state = 0
        b.next_u32()
        b.state = (b.state + 0x853C49E6748FEA9D) & M64
        b.next_u32()
        assert [a.next_u32() for _ in range(4)] == [b.next_u32() for _ in range(4)]


def test_step_rng_matches_oracle_and_next_f32(oracle):
    # rng.rs:224-232 (deterministic, seeds differ) and next_f32 = (u >> 8) * 2^-24
    for seed in (7, 42, 43):
        a, o = rng.StepRng(seed), oracle.StepRng(seed)
        for _ in range(6):
            assert a.next_u32() == o.next_u32()
        a, b = rng.StepRng(seed), rng.StepRng(seed)
        for _ in range(6):
            u = b.next_u32()
            f = a.next_f32()
            assert f.dtype == np.float32 and f == np.float32((u >> 8) * 2.0**-24)
            assert 0.0 <= f < 1.0
    assert rng.StepRng(42).next_u32() != rng.StepRng(43).next_u32()
    c = rng.StepRng(42)
    c.next_u32()
    d = c.clone()
    assert c.next_u32() == d.next_u32()


def test_nano_lcg_first_draw():
    # crates/moss-tts/src/nano/sampling.rs:171: seed 42, first draw 0.252345...
    n = rng.NanoLcg(42)
    u = n.next_unit()
    # state 42 * 1664525 + 1013904223 = 1083814273; 1083814273 >> 8 = 4233649
    assert n.state == 1083814273
    assert u == 4233649 / 16777216.0
    assert abs(u - 0.25234514) < 1e-8


def test_unit_f64_range_and_determinism():
    a, b = rng.unit_f64(5, 1000), rng.unit_f64(5, 1000)
    assert np.array_equal(a, b) and a.dtype == np.float64
    assert (a >= 0).all() and (a < 1).all()
    # (u64 >> 11) * 2^-53: every value is a multiple of 2^-53
    assert np.all(np.ldexp(a, 53) == np.floor(np.ldexp(a, 53)))
