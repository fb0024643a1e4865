"""neurogrid_amd - gfx950 (MI355X) build of NeuroGrid's per-layer kernel set.

The product is ``lib/libgpu_engine.so``: hand-written HIP kernels behind the C
ABI of the reference's ``libgpu_engine.so`` (declared in ``include/*.h``).
This package holds their sources (``csrc/``), the build (``build.py``), the
ctypes loader (``_lib.py``), a restatement of the reference's Go wrappers
(``bindings.py``) and raw device buffers (``device.py``).
"""

__all__ = ["build", "bindings", "device"]
