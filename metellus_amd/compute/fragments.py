"""Codegen core: LDS access records, kernel context, barrier/alias fragments
and the engine that renders a fragment list into one HIP kernel for gfx950.

Fragment protocol (kept from the reference, src/compute/fragments.py:12-142):
any object with ``name``, ``kind``, ``render(ctx) -> str`` and
``tgmem_accesses``; optionally ``sub_fragments`` (walked by the LDS lifetime
pass) and ``is_tgmem_barrier``.

Rendered kernel layout::

    <device header: metellus_amd/csrc/mt_device.h>
    extern "C" __global__ void __launch_bounds__(NT) fn(<buffers...>, const mt_dims dims) {
        const unsigned M = dims.v[0];  ...          // runtime dims, by value
        <preamble>
        __shared__ alignas(16) float X_tile[..][..];  // LDS declarations
        <fragment bodies in order>
    }

Dims travel in the kernel-argument segment as a fixed 16-word struct
(``mt_dims``) at ``dims_buffer_index`` (default: after the buffers), instead of
the per-launch dims buffer the reference allocates (reference:
src/runtime/program.py:186).  A kernel with ``workspace_bytes`` (stream-K
matmuls) takes one more parameter, ``float* mt_ws``, after everything else;
the runtime passes the shim's workspace there.
"""

from __future__ import annotations

import functools
import math
import os
import re
import textwrap
from dataclasses import dataclass
from typing import Any, Literal

KernelFragment = Any
TgmemAccessKind = Literal["read", "write", "readwrite"]

MAX_DIMS = 16  # words in the by-value ``mt_dims`` kernel argument


@dataclass(frozen=True)
class TgmemAccess:
    """One named LDS object touched by a fragment.  ``shape`` is the logical
    array shape (2-D or 3-D for double-buffered tiles); ``size_floats`` its
    element count."""

    name: str
    access: TgmemAccessKind
    size_floats: int
    shape: tuple[int, ...]


@dataclass(frozen=True)
class CodegenContext:
    function_name: str
    buffers: tuple[str, ...]
    dims: tuple[str, ...]
    tg_x: int
    tg_y: int
    threadgroup_decls: tuple[str, ...] = ()
    helpers: tuple[str, ...] = ()
    preamble: tuple[str, ...] = ()
    dims_buffer_index: int | None = None
    tg_z: int = 1
    batched: bool = False
    # Bytes of device workspace the kernel takes as its last parameter
    # (``float* mt_ws``, after the dims); 0 = none.
    workspace_bytes: int = 0
    # The kernel indexes its workspace by blockIdx.z, so its batched variant
    # shares one workspace (workspace_bytes covers the batch it was built for).
    workspace_batched: bool = False

    @property
    def num_threads(self) -> int:
        return self.tg_x * self.tg_y * self.tg_z


@dataclass(frozen=True)
class BarrierFragment:
    """Workgroup barrier; also orders LDS accesses (``s_barrier`` with the
    LDS counter drained)."""

    name: str = "barrier"
    kind: str = "barrier"

    def render(self, ctx: CodegenContext) -> str:
        return "__syncthreads();"

    @property
    def is_tgmem_barrier(self) -> bool:
        return True

    @property
    def tgmem_accesses(self) -> tuple[TgmemAccess, ...]:
        return ()


def lds_pointer_type(name: str, shape: tuple[int, ...]) -> str:
    """``float (*name)[d1][d2]`` -- a pointer that indexes like an array of
    ``shape``."""
    inner = "".join(f"[{d}]" for d in shape[1:])
    return f"float (*{name}){inner}" if inner else f"float* {name}"


@dataclass(frozen=True)
class AliasFragment:
    """Re-type a shared LDS storage block as tenant ``new_name`` of shape
    ``new_shape``.  Emitted by the aliasing rewriter where two LDS objects
    with disjoint lifetimes share storage (reference semantics:
    src/compute/fragments.py:50-93).  A barrier must separate the previous
    tenant's last access from the new tenant's first access; the fragment
    emits one unless the template already placed one right before it."""

    old_name: str
    new_name: str
    new_shape: tuple[int, ...]
    preceded_by_barrier: bool
    name: str = "alias"
    kind: str = "alias"

    def render(self, ctx: CodegenContext) -> str:
        ptr = lds_pointer_type(self.new_name, self.new_shape)
        cast_t = lds_pointer_type("", self.new_shape)
        line = f"{ptr} = reinterpret_cast<{cast_t}>({self.old_name});"
        if self.preceded_by_barrier:
            return line
        return f"__syncthreads();\n{line}"

    @property
    def tgmem_accesses(self) -> tuple[TgmemAccess, ...]:
        return ()


def lds_decl(name: str, shape: tuple[int, ...]) -> str:
    """Canonical LDS declaration parsed by the aliasing pass."""
    dims = "".join(f"[{d}]" for d in shape)
    return f"__shared__ alignas(16) float {name}{dims};"


@functools.lru_cache(maxsize=1)
def device_header() -> str:
    """The hand-written gfx950 device library prepended to every kernel."""
    path = os.path.join(os.path.dirname(os.path.dirname(__file__)), "csrc", "mt_device.h")
    with open(path, encoding="utf-8") as f:
        return f.read()


_PARAM_RE = re.compile(r"^\s*(const\s+)?float\s*\*\s*__restrict__\s+(\w+)\s*$")


def batched_params(buffers: tuple[str, ...]) -> tuple[list[str], list[str]]:
    """Batched variant of a kernel signature: every ``[const] float*
    __restrict__ g_X`` parameter becomes a device table of per-program
    pointers ``g_X_tab`` and the body starts by picking entry ``blockIdx.z``.

    The table entries are typed as global-address-space pointers: a pointer
    read from memory is otherwise generic, every access through it becomes a
    flat instruction, and flat loads also count against the LDS wait counter,
    so each LDS read of a pipelined mainloop would wait for the next chunk's
    global loads."""
    params, picks = [], []
    for decl in buffers:
        m = _PARAM_RE.match(decl)
        if m is None:
            raise ValueError(f"cannot batch kernel parameter {decl!r}")
        const, name = m.group(1) or "", m.group(2)
        params.append(f"{const}MT_GLOBAL float* const* __restrict__ {name}_tab")
        picks.append(f"{const}float* __restrict__ {name} = ({const}float*){name}_tab[blockIdx.z];")
    return params, picks


class CodegenEngine:
    def render(self, fragments: list[KernelFragment], ctx: CodegenContext) -> str:
        dims_index = ctx.dims_buffer_index if ctx.dims_buffer_index is not None else len(ctx.buffers)
        if len(ctx.dims) > MAX_DIMS:
            raise ValueError(f"at most {MAX_DIMS} dims per kernel; got {len(ctx.dims)}")
        if ctx.batched:
            params, picks = batched_params(ctx.buffers)
        else:
            params, picks = list(ctx.buffers), []
        params.insert(dims_index, "const mt_dims dims")
        if ctx.workspace_bytes:
            if ctx.batched and not ctx.workspace_batched:
                raise ValueError(f"{ctx.function_name}: a kernel with a workspace is not batched")
            params.append("float* mt_ws")
        body_parts = [
            *picks,
            self._dim_decls(ctx.dims),
            *ctx.preamble,
            *ctx.threadgroup_decls,
            *(fragment.render(ctx) for fragment in fragments),
        ]
        body = "\n".join(p for p in body_parts if p.strip())
        helpers = "\n".join(h.strip() for h in ctx.helpers if h.strip())
        sep = ",\n    "
        return (
            f"{device_header()}\n"
            f"{helpers}\n"
            f'extern "C" __global__ void __launch_bounds__({ctx.num_threads})\n'
            f"{ctx.function_name}(\n    {sep.join(params)}\n) {{\n"
            f"{textwrap.indent(body.strip(), '    ')}\n"
            f"}}\n"
        )

    def render_many(self, stages: list[tuple[list[KernelFragment], CodegenContext]]) -> tuple[str, ...]:
        return tuple(self.render(f, c) for f, c in stages)

    @staticmethod
    def _dim_decls(dims: tuple[str, ...]) -> str:
        return "\n".join(f"const unsigned {name} = dims.v[{i}];" for i, name in enumerate(dims))


def prod(shape: tuple[int, ...]) -> int:
    return math.prod(shape) if shape else 1
