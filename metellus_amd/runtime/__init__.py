"""Runtime steps over the native HIP shim.  ``Buffer`` (and the shim) load
lazily, so importing the pipeline needs no GPU."""

from metellus_amd.runtime.program import (
    Allocate,
    Dispatch,
    Download,
    Env,
    Fill,
    Free,
    FromNumpy,
    Kernel,
    Runtime,
    RuntimeFragment,
    Upload,
)


def __getattr__(name):
    if name == "Buffer":
        from metellus_amd.runtime.buffer import Buffer

        return Buffer
    raise AttributeError(f"module {__name__!r} has no attribute {name!r}")


__all__ = [
    "Allocate",
    "Buffer",
    "Dispatch",
    "Download",
    "Env",
    "Fill",
    "Free",
    "FromNumpy",
    "Kernel",
    "Runtime",
    "RuntimeFragment",
    "Upload",
]
