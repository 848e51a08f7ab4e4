"""ctypes wrapper over the native shim ``libmetellus_hip.so``.

Exposes the seven functions of the reference's native module
(reference: src/metal_backend.mm:253-261) with the same names, arguments
and error behaviour (failures raise ``RuntimeError``):

    create_buffer(nbytes) -> int          release_buffer(handle) -> bool
    buffer_size(handle) -> int            write_buffer(handle, ndarray)
    read_buffer(handle, ndarray)          fill_buffer(handle, value)
    run_kernel(source, function_name, buffers, grid, threads, *, dims=(), dims_slot=None)
        -> {"time_ms": float}

plus the finer-grained ``compile_kernel`` / ``launch`` used by the runtime.

The library is built in-tree by ``__graft_entry__.build()`` (hipcc, gfx950).
There is no fallback: if the library or a GPU is missing, calls fail loudly.
"""

from __future__ import annotations

import ctypes
import os
import threading

import numpy as np

_LIB_PATH = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "_lib", "libmetellus_hip.so")

# Symbols declared in include/metellus_hip.h (checked by the CPU test suite).
EXPORTED_SYMBOLS = (
    "mt_last_error",
    "mt_init",
    "mt_device_count",
    "mt_device_info",
    "mt_device_pci",
    "mt_alloc",
    "mt_free",
    "mt_trim",
    "mt_cache_info",
    "mt_alloc_stats",
    "mt_size",
    "mt_device_ptr",
    "mt_write",
    "mt_read",
    "mt_fill",
    "mt_host_alloc",
    "mt_host_free",
    "mt_compile",
    "mt_compile_only",
    "mt_launch",
    "mt_launch_noalloc",
    "mt_mark",
    "mt_mark_elapsed",
    "mt_sync",
    "mt_cache_stats",
    "mt_workspace",
    "mt_workspace_check",
)

_lib = None
_lock = threading.Lock()

_u64 = ctypes.c_uint64
_u32p = ctypes.POINTER(ctypes.c_uint32)


def library_path() -> str:
    return _LIB_PATH


def _load():
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not os.path.exists(_LIB_PATH):
            raise RuntimeError(
                f"native HIP shim not built: {_LIB_PATH} is missing "
                "(run `python -c 'import __graft_entry__ as g; g.build()'` at the repo root)"
            )
        lib = ctypes.CDLL(_LIB_PATH)
        sig = {
            "mt_last_error": ([], ctypes.c_char_p),
            "mt_init": ([], ctypes.c_int),
            "mt_device_count": ([ctypes.POINTER(ctypes.c_int)], ctypes.c_int),
            "mt_device_info": (
                [ctypes.c_char_p, ctypes.c_size_t, ctypes.POINTER(ctypes.c_int), ctypes.POINTER(ctypes.c_int)],
                ctypes.c_int,
            ),
            "mt_device_pci": (
                [ctypes.c_char_p, ctypes.c_size_t, ctypes.POINTER(ctypes.c_int), ctypes.POINTER(_u64)],
                ctypes.c_int,
            ),
            "mt_alloc": ([ctypes.c_size_t, ctypes.POINTER(_u64)], ctypes.c_int),
            "mt_free": ([_u64, ctypes.POINTER(ctypes.c_int)], ctypes.c_int),
            "mt_trim": ([], ctypes.c_int),
            "mt_cache_info": ([ctypes.POINTER(ctypes.c_size_t), ctypes.POINTER(ctypes.c_size_t)], ctypes.c_int),
            "mt_alloc_stats": (
                [ctypes.POINTER(_u64), ctypes.POINTER(_u64), ctypes.POINTER(_u64), ctypes.POINTER(ctypes.c_size_t)],
                ctypes.c_int,
            ),
            "mt_size": ([_u64, ctypes.POINTER(ctypes.c_size_t)], ctypes.c_int),
            "mt_device_ptr": ([_u64, ctypes.POINTER(_u64)], ctypes.c_int),
            "mt_write": ([_u64, ctypes.c_void_p, ctypes.c_size_t], ctypes.c_int),
            "mt_read": ([_u64, ctypes.c_void_p, ctypes.c_size_t], ctypes.c_int),
            "mt_fill": ([_u64, ctypes.c_uint8], ctypes.c_int),
            "mt_host_alloc": ([ctypes.c_size_t, ctypes.POINTER(ctypes.c_void_p)], ctypes.c_int),
            "mt_host_free": ([ctypes.c_void_p], ctypes.c_int),
            "mt_compile": ([ctypes.c_char_p, ctypes.c_char_p, ctypes.c_char_p, ctypes.POINTER(_u64)], ctypes.c_int),
            "mt_compile_only": (
                [ctypes.c_char_p, ctypes.c_char_p, ctypes.c_char_p, ctypes.POINTER(ctypes.c_size_t)],
                ctypes.c_int,
            ),
            "mt_launch": (
                [_u64, ctypes.POINTER(_u64), ctypes.c_int, _u32p, ctypes.c_int, ctypes.c_int, _u32p, _u32p,
                 ctypes.c_int, ctypes.POINTER(ctypes.c_float)],
                ctypes.c_int,
            ),
            "mt_launch_noalloc": (
                [_u64, ctypes.POINTER(_u64), ctypes.c_int, _u32p, ctypes.c_int, ctypes.c_int, _u32p, _u32p,
                 ctypes.c_size_t, _u32p],
                ctypes.c_int,
            ),
            "mt_mark": ([ctypes.c_int], ctypes.c_int),
            "mt_mark_elapsed": ([ctypes.c_int, ctypes.c_int, ctypes.POINTER(ctypes.c_float)], ctypes.c_int),
            "mt_sync": ([], ctypes.c_int),
            "mt_cache_stats": ([ctypes.POINTER(_u64), ctypes.POINTER(_u64)], ctypes.c_int),
            "mt_workspace": ([ctypes.c_size_t, ctypes.POINTER(_u64)], ctypes.c_int),
            "mt_workspace_check": ([ctypes.POINTER(ctypes.c_uint32)], ctypes.c_int),
        }
        for name, (args, res) in sig.items():
            fn = getattr(lib, name)
            fn.argtypes = args
            fn.restype = res
        _lib = lib
        return lib


def _check(rc: int) -> None:
    if rc != 0:
        msg = _load().mt_last_error().decode("utf-8", "replace")
        raise RuntimeError(msg)


def library():
    """The loaded ctypes library (raises if it was not built)."""
    return _load()


# ---------------------------------------------------------------------------
# device
# ---------------------------------------------------------------------------


def device_count() -> int:
    n = ctypes.c_int(0)
    _check(_load().mt_device_count(ctypes.byref(n)))
    return n.value


def device_info() -> dict:
    arch = ctypes.create_string_buffer(128)
    cus = ctypes.c_int(0)
    clk = ctypes.c_int(0)
    _check(_load().mt_device_info(arch, 128, ctypes.byref(cus), ctypes.byref(clk)))
    return {"arch": arch.value.decode(), "cu_count": cus.value, "clock_khz": clk.value}


def device_pci() -> dict:
    """PCI bus id, memory clock (kHz) and memory size (bytes) of device 0."""
    bus = ctypes.create_string_buffer(64)
    mclk = ctypes.c_int(0)
    mem = _u64(0)
    _check(_load().mt_device_pci(bus, 64, ctypes.byref(mclk), ctypes.byref(mem)))
    return {"pci_bus_id": bus.value.decode(), "memory_clock_khz": mclk.value, "memory_bytes": mem.value}


def synchronize() -> None:
    _check(_load().mt_sync())


def mark(slot: int) -> None:
    """Record timing marker ``slot`` (0..15) on the shim's stream."""
    _check(_load().mt_mark(int(slot)))


def mark_elapsed(first: int, last: int) -> float:
    """Wait for marker ``last``; GPU milliseconds from ``first`` to ``last``."""
    ms = ctypes.c_float(0.0)
    _check(_load().mt_mark_elapsed(int(first), int(last), ctypes.byref(ms)))
    return float(ms.value)


def cache_stats() -> tuple[int, int]:
    c, h = _u64(0), _u64(0)
    _check(_load().mt_cache_stats(ctypes.byref(c), ctypes.byref(h)))
    return c.value, h.value


# ---------------------------------------------------------------------------
# buffers (reference names)
# ---------------------------------------------------------------------------


def create_buffer(nbytes: int) -> int:
    h = _u64(0)
    _check(_load().mt_alloc(int(nbytes), ctypes.byref(h)))
    return h.value


def release_buffer(handle: int) -> bool:
    existed = ctypes.c_int(0)
    _check(_load().mt_free(int(handle), ctypes.byref(existed)))
    return bool(existed.value)


def trim() -> None:
    """Return the shim's cached device blocks (freed buffers kept for reuse)
    to the driver."""
    _check(_load().mt_trim())


def device_cache_info() -> tuple[int, int]:
    """(bytes, blocks) held in the shim's device block cache."""
    nb, nk = ctypes.c_size_t(0), ctypes.c_size_t(0)
    _check(_load().mt_cache_info(ctypes.byref(nb), ctypes.byref(nk)))
    return nb.value, nk.value


def alloc_stats() -> dict:
    """Allocations the shim has requested from the runtime so far
    (``device_allocs``: hipMallocAsync, ``host_allocs``: hipHostMalloc), the
    buffers its registry holds (``live_buffers``, the workspace included) and
    the workspace's size (``workspace_bytes``, 0 before the first stream-K
    launch)."""
    d, h, n = _u64(0), _u64(0), _u64(0)
    w = ctypes.c_size_t(0)
    _check(_load().mt_alloc_stats(ctypes.byref(d), ctypes.byref(h), ctypes.byref(n), ctypes.byref(w)))
    return {"device_allocs": d.value, "host_allocs": h.value, "live_buffers": n.value, "workspace_bytes": w.value}


def buffer_size(handle: int) -> int:
    n = ctypes.c_size_t(0)
    _check(_load().mt_size(int(handle), ctypes.byref(n)))
    return n.value


def device_address(handle: int) -> int:
    a = _u64(0)
    _check(_load().mt_device_ptr(int(handle), ctypes.byref(a)))
    return a.value


def _handle_of(item) -> int:
    if hasattr(item, "handle"):
        return int(item.handle)
    if isinstance(item, (int, np.integer)):
        return int(item)
    raise TypeError(f"expected a Buffer or an int handle; got {type(item).__name__}")


def write_buffer(handle, data: np.ndarray) -> None:
    arr = np.ascontiguousarray(data)
    _check(_load().mt_write(_handle_of(handle), arr.ctypes.data_as(ctypes.c_void_p), arr.nbytes))


def read_buffer(handle, out: np.ndarray) -> None:
    if not out.flags["C_CONTIGUOUS"]:
        raise ValueError("read_buffer: destination must be C-contiguous")
    _check(_load().mt_read(_handle_of(handle), out.ctypes.data_as(ctypes.c_void_p), out.nbytes))


def host_alloc(nbytes: int) -> int:
    """Page-locked host memory (pooled); returns its address."""
    p = ctypes.c_void_p(0)
    _check(_load().mt_host_alloc(int(nbytes), ctypes.byref(p)))
    return int(p.value)


def host_free(address: int) -> None:
    _check(_load().mt_host_free(ctypes.c_void_p(int(address))))


def fill_buffer(handle, value: int) -> None:
    if not 0 <= int(value) <= 255:
        raise ValueError(f"fill value must be in [0, 255]; got {value}")
    _check(_load().mt_fill(_handle_of(handle), int(value)))


# ---------------------------------------------------------------------------
# kernels
# ---------------------------------------------------------------------------


def compile_kernel(source: str, function_name: str, options: str = "") -> int:
    """hiprtc-compile (cached) and load; returns a kernel handle."""
    k = _u64(0)
    _check(_load().mt_compile(source.encode(), function_name.encode(), options.encode(), ctypes.byref(k)))
    return k.value


def compile_only(source: str, options: str = "", target: str = "gfx950") -> int:
    """hiprtc-compile without a device; returns the code-object size."""
    n = ctypes.c_size_t(0)
    _check(_load().mt_compile_only(source.encode(), options.encode(), target.encode(), ctypes.byref(n)))
    return n.value


def workspace_handle(nbytes: int) -> int:
    """Handle of the shim's device workspace (at least ``nbytes``)."""
    h = _u64(0)
    _check(_load().mt_workspace(int(nbytes), ctypes.byref(h)))
    return h.value


def check_workspace() -> None:
    """Raise if a stream-K workgroup gave up waiting for a partial tile since
    the last check (the results of that launch are invalid)."""
    err = ctypes.c_uint32(0)
    _check(_load().mt_workspace_check(ctypes.byref(err)))
    if err.value:
        raise RuntimeError(
            "stream-K matmul: a workgroup gave up waiting for another workgroup's partial tile; "
            "the results of that launch are invalid (the workspace flags were reset)"
        )


def launch(
    kernel: int,
    buffers,
    dims,
    dims_slot: int,
    grid,
    threads,
    timed: bool = False,
    workspace: int = 0,
) -> float | None:
    """Launch ``kernel``; buffers are handles (or objects with ``.handle``).
    ``workspace`` > 0: the kernel takes the shim's workspace (at least that
    many bytes) as its last parameter.  Returns the kernel time in ms when
    ``timed``."""
    handles = [_handle_of(b) for b in buffers]
    if workspace:
        handles.append(workspace_handle(workspace))
    nb = len(handles)
    bufs = (_u64 * max(nb, 1))(*handles)
    dims_l = [int(d) for d in dims]
    for d in dims_l:
        if not 0 <= d < 2**32:
            raise ValueError(f"dim value {d} does not fit in uint32")
    dims_a = (ctypes.c_uint32 * max(len(dims_l), 1))(*dims_l)
    grid_a = (ctypes.c_uint32 * 3)(*[int(g) for g in grid])
    block_a = (ctypes.c_uint32 * 3)(*[int(t) for t in threads])
    ms = ctypes.c_float(0.0)
    _check(
        _load().mt_launch(
            kernel, bufs, nb, dims_a, len(dims_l), int(dims_slot), grid_a, block_a, 1 if timed else 0,
            ctypes.byref(ms),
        )
    )
    return float(ms.value) if timed else None


def launch_noalloc(kernel: int, buffers, dims, dims_slot: int, grid, threads, scratch: int = 0,
                   wait: bool = True) -> int | None:
    """``mt_launch_noalloc``: launch without allocating; a stream-K kernel
    (``scratch`` = its ``workspace_bytes``) gets the library's static scratch
    as its last parameter.  ``wait``: synchronise and return the scratch's
    error word (0 unless a stream-K wait gave up); otherwise None."""
    handles = [_handle_of(b) for b in buffers]
    nb = len(handles)
    bufs = (_u64 * max(nb, 1))(*handles)
    dims_l = [int(d) for d in dims]
    for d in dims_l:
        if not 0 <= d < 2**32:
            raise ValueError(f"dim value {d} does not fit in uint32")
    dims_a = (ctypes.c_uint32 * max(len(dims_l), 1))(*dims_l)
    grid_a = (ctypes.c_uint32 * 3)(*[int(g) for g in grid])
    block_a = (ctypes.c_uint32 * 3)(*[int(t) for t in threads])
    err = ctypes.c_uint32(0)
    _check(
        _load().mt_launch_noalloc(
            kernel, bufs, nb, dims_a, len(dims_l), int(dims_slot), grid_a, block_a, int(scratch),
            ctypes.byref(err) if wait else None,
        )
    )
    return int(err.value) if wait else None


def init() -> None:
    """Select the device and create the shim's stream (``mt_init``)."""
    _check(_load().mt_init())


def _check_slot(item) -> bool:
    """Validate one ``run_kernel`` slot; True when it is an array (a one-shot
    buffer with write-back).  Like the reference (src/metal_backend.mm:153-176):
    an object with ``.handle`` or an int is a persistent buffer, an ndarray a
    transient one."""
    if hasattr(item, "handle") or isinstance(item, (int, np.integer)):
        return False
    if not isinstance(item, np.ndarray):
        raise TypeError(f"run_kernel: a slot is a Buffer, an int handle or an ndarray; got {type(item).__name__}")
    if not item.flags["C_CONTIGUOUS"] or not item.flags["WRITEABLE"]:
        # the reference's binding refuses read-only arrays too
        raise ValueError("run_kernel: an array slot must be C-contiguous and writeable (its contents are written back in place)")
    return True


def run_kernel(source: str, function_name: str, buffers, grid, threads, *, dims=(), dims_slot=None) -> dict:
    """Compile (cached) + launch + wait, returning ``{"time_ms": t}`` like the
    reference (reference: src/metal_backend.mm:178-249).  ``buffers`` holds
    one slot per kernel buffer parameter, in order: a Buffer, an int handle,
    or a NumPy array, which is uploaded to a one-shot device buffer and, once
    the kernel has finished, copied back into the array (slots in order) --
    so an output array receives the kernel's result (reference:
    src/metal_backend.mm:235-239).  Slots are checked before anything is
    compiled or allocated.  ``dims`` are passed by value at ``dims_slot``
    (default: after the buffers)."""
    items = list(buffers)
    is_array = [_check_slot(item) for item in items]
    k = compile_kernel(source, function_name)
    handles: list[int] = []
    transient: list[tuple[int, np.ndarray]] = []
    try:
        for item, arr in zip(items, is_array):
            if not arr:
                handles.append(_handle_of(item))
                continue
            # a zero-size array still binds a valid (unused) pointer
            h = create_buffer(max(int(item.nbytes), 4))
            transient.append((h, item))
            handles.append(h)
            if item.nbytes:
                write_buffer(h, item)
        slot = len(handles) if dims_slot is None else int(dims_slot)
        # a timed launch waits for the kernel, so the write-backs read its result
        t = launch(k, handles, dims, slot, grid, threads, timed=True)
        for h, target in transient:
            if target.nbytes:
                read_buffer(h, target)
    finally:
        for h, _ in transient:
            release_buffer(h)
    return {"time_ms": t}
