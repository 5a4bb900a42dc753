"""zeno_amd: Lulzx/zeno's batched rigid-body physics step, built for AMD MI355X (gfx950).

The step runs as hand-written HIP kernels behind libzeno.so, whose C ABI matches the
reference's (include/zeno.h). This package holds the build script, the ctypes bindings and
the Python ZenoWorld mirror of the reference's python/zeno/_ffi.py.
"""
from pathlib import Path

from .world import CONTACT_DTYPE, ZenoWorld, is_metal_available, version  # noqa: F401

ASSETS = Path(__file__).resolve().parent / "assets"

__all__ = ["ZenoWorld", "CONTACT_DTYPE", "version", "is_metal_available", "ASSETS"]
