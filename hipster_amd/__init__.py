"""hipster_amd: MI355X (gfx950) quantized-matmul hot path of dzannotti/hipster.

``hipster_amd.qmm`` mirrors the reference's engine/kernels call surface over the C ABI in
include/hipster_qmm.h; ``hipster_amd.synth`` makes the seeded synthetic GGUF tensors the tests and
the benchmark run on.
"""
from . import _lib  # noqa: F401

__all__ = ["qmm", "synth"]
