"""loom_amd -- MI355X (gfx950) runtime for LoomFormer's fused-kernel inference path.

* ``_lib``   ctypes binding of libloom_hip.so (the C ABI in include/loom_hip.h)
* ``ops``    torch-level mirror of the reference's extension functions
* ``engine`` the batched greedy decode (Model.step) on those kernels
"""
from . import _lib, ops  # noqa: F401

__all__ = ["_lib", "ops"]
