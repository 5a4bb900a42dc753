"""zeno_amd: Lulzx/zeno's batched rigid-body physics step, built for AMD MI355X (gfx950).

The step runs as hand-written HIP kernels behind libzeno.so, whose C ABI matches the
reference's (include/zeno.h). This package holds the build script, the ctypes bindings,
the ZenoWorld mirror of the reference's python/zeno/_ffi.py, the batched ZenoEnv / make of
python/zeno/env.py and the Gymnasium-style environments of python/zeno/gym (zeno_amd.gym).
"""
from pathlib import Path

from .world import CONTACT_DTYPE, ZenoWorld, is_metal_available, version  # noqa: F401
from .env import ZenoEnv, make  # noqa: F401

__version__ = "0.1.0"
ASSETS = Path(__file__).resolve().parent / "assets"


def info() -> dict:
    """Version and capability information (python/zeno/__init__.py:113-125)."""
    return {"version": __version__, "metal_available": is_metal_available(), "library_version": version()}


__all__ = ["ZenoWorld", "ZenoEnv", "make", "CONTACT_DTYPE", "version", "is_metal_available", "info", "ASSETS"]
