"""MI355X-native (gfx950) HIP implementation of Tenzo's quantized decode hot path.

The compute lives in ``libtenzo_hip.so`` (HIP kernels + C ABI, sources in
``csrc/``). This package holds the host-side mirror of the reference operator
interface (``ops``), the engine binding (``engine``), load-time weight formats
(``formats``) and seeded synthetic inputs (``synth``).
"""
from . import formats, synth  # noqa: F401

__all__ = ["formats", "synth"]
