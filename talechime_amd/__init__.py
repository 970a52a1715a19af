"""MI355X-native per-step token sampler for talechime's autoregressive TTS crates.

The compute path is ``libtalechime_hip.so`` (hand-written HIP kernels for
gfx950 behind a C ABI, declared in ``include/talechime_hip.h``).  The Python
modules mirror the reference crates' sampler interfaces on top of it:

  talechime_amd.qwen        crates/qwen3-tts/src/generation/{sampling,tts}.rs and the
                            talker's caller chain (synthesis.rs)
  talechime_amd.cosyvoice3  crates/cosyvoice3/src/llm.rs (sample, RAS)
  talechime_amd.indextts    crates/indextts/src/generation.rs (processors + draw,
                            beam-sample and beam-search steps, the host scorer)
  talechime_amd.moss        crates/moss-tts/src/{sampling,nano/sampling}.rs

They sit on ``talechime_amd.sampler`` (the ctypes binding, torch tensors in and
out) and draw their uniforms from ``talechime_amd.rng``.

Importing the package does not load the library; the first sampler call does,
and raises if the library is missing.
"""
__all__ = ["rng", "synth", "sampler", "qwen", "cosyvoice3", "indextts", "moss", "beam"]
