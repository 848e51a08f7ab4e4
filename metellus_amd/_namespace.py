"""Map the reference's top-level module names onto this package.

The reference lays its packages out flat under ``src/`` and callers write
``from orchestrator import Operations`` or ``from runtime import Dispatch``.
Here the same modules live under ``metellus_amd.*``.  The finder below makes
``orchestrator.fusion`` *the same module object* as
``metellus_amd.orchestrator.fusion`` (not a second copy), so ``isinstance``
checks and monkeypatching behave identically through either name.
"""

from __future__ import annotations

import importlib
import importlib.abc
import importlib.machinery
import importlib.util
import sys

# reference top-level name -> module path inside this package
_ALIASES = {
    "orchestrator": "metellus_amd.orchestrator",
    "compute": "metellus_amd.compute",
    "memory": "metellus_amd.memory",
    "runtime": "metellus_amd.runtime",
    "api": "metellus_amd.api",
    # the reference's native module; here it is the ctypes wrapper over the HIP shim
    "metal_backend": "metellus_amd.runtime.hip_backend",
}


def _target_for(fullname: str) -> str | None:
    head, _, rest = fullname.partition(".")
    base = _ALIASES.get(head)
    if base is None:
        return None
    return f"{base}.{rest}" if rest else base


class _AliasLoader(importlib.abc.Loader):
    def __init__(self, target: str) -> None:
        self._target = target
        self._real_spec = None

    def create_module(self, spec):  # noqa: D401 - importlib protocol
        module = importlib.import_module(self._target)
        self._real_spec = module.__spec__
        return module

    def exec_module(self, module) -> None:
        # The real module was executed under its own name already; importlib
        # overwrote its __spec__ with the alias spec, so put the real one back
        # (lazy relative imports inside the module resolve against it).
        if self._real_spec is not None:
            module.__spec__ = self._real_spec


class _AliasFinder(importlib.abc.MetaPathFinder):
    def find_spec(self, fullname, path=None, target=None):
        real = _target_for(fullname)
        if real is None:
            return None
        try:
            real_spec = importlib.util.find_spec(real)
        except ModuleNotFoundError:
            return None
        if real_spec is None:
            return None
        spec = importlib.machinery.ModuleSpec(
            fullname,
            _AliasLoader(real),
            is_package=real_spec.submodule_search_locations is not None,
        )
        return spec


_FINDER = _AliasFinder()


def install_reference_namespace() -> None:
    """Make ``orchestrator``, ``compute``, ``memory``, ``runtime``, ``api`` and
    ``metal_backend`` importable as aliases of this package's modules.
    Idempotent."""
    if _FINDER not in sys.meta_path:
        sys.meta_path.insert(0, _FINDER)
