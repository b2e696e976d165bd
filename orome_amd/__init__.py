"""orome_amd: MI355X (gfx950) implementation of Orome's MoE feed-forward path.

The compute lives in liborome_moe.so (HIP kernels behind a C ABI, see
include/orome_moe.h); this package binds it.  Importing fails loudly if the
library has not been built (`python orome_amd/build.py`).
"""
from ._lib import lib, OromeError  # noqa: F401
from .moe import Context, DeviceBuffer, MoEModel, make_spec, synth_gguf, synth_normal  # noqa: F401

__all__ = ["lib", "OromeError", "Context", "DeviceBuffer", "MoEModel", "make_spec", "synth_gguf",
           "synth_normal"]
