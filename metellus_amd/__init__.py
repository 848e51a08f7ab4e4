"""metellus_amd — an MI355X (gfx950) backend for the Metellus fragment compiler.

The Python pipeline keeps the reference's API:

    ops.build() -> fuse -> assemble -> alias_group -> schedule -> Runtime.run()

Fragments emit HIP C++ for gfx950; the native shim (``csrc/mt_shim.cpp``,
C ABI declared in ``include/metellus_hip.h``) compiles each generated kernel
with hiprtc, caches the code object and launches it on one HIP stream.

Reference callers import the top-level package names ``orchestrator``,
``compute``, ``memory``, ``runtime``, ``api`` (the reference runs with
``PYTHONPATH=src``).  :func:`install_reference_namespace` makes those names
resolve to the subpackages of this package, so such code runs unchanged.
"""

from __future__ import annotations

__version__ = "0.1.0"

from metellus_amd._namespace import install_reference_namespace  # noqa: E402

__all__ = ["install_reference_namespace", "__version__"]
