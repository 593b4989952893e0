"""janus_amd -- MI355X-native (gfx950) decode hot path of janus-engine.

The product is libjanus_hip.so (hand-written HIP kernels behind the C ABI in
include/janus_hip.h and the C++ decode driver in include/janus_model.h).
This package builds it (`python -m janus_amd.build`), binds it with ctypes
and mirrors the reference's operator API (`janus_amd.ops`) and model API
(`janus_amd.model`) on top.
"""
from . import _lib  # noqa: F401

__all__ = ["_lib", "ops", "model", "synth", "build"]


def load():
    """Load libjanus_hip.so (raises if it has not been built)."""
    return _lib.load()
