"""MI355X (gfx950) implementation of instantcua's Qwen3-VL text-decoder token loop.

``engine`` mirrors the reference ``Engine`` over the C ABI of ``include/icua.h``;
``modelfile`` and ``synth`` write the ``.icua`` model layout and seeded synthetic workloads.
"""
__all__ = ["engine", "modelfile", "synth", "build"]
