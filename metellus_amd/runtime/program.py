"""Host-side program steps and the ``Runtime`` that runs them in order
(reference: src/runtime/program.py:1-215).  Same step types and env
conventions; kernels are HIP sources compiled once per process by the
native shim and launched on its stream."""

from __future__ import annotations

from dataclasses import dataclass, field
from typing import Any, Protocol

import numpy as np

from metellus_amd.compute.fragments import CodegenContext, CodegenEngine

Env = dict[str, Any]


class RuntimeFragment(Protocol):
    def execute(self, env: Env) -> None: ...


def _buffer_cls():
    from metellus_amd.runtime.buffer import Buffer

    return Buffer


@dataclass(frozen=True)
class Allocate:
    name: str
    nbytes: int

    def execute(self, env: Env) -> None:
        if self.name in env:
            raise KeyError(f"Allocate: key {self.name!r} already in env")
        env[self.name] = _buffer_cls()(self.nbytes)


@dataclass(frozen=True)
class Free:
    name: str

    def execute(self, env: Env) -> None:
        env.pop(self.name).release()


@dataclass(frozen=True)
class Upload:
    name: str
    source: np.ndarray

    def execute(self, env: Env) -> None:
        env[self.name].write(self.source)


@dataclass(frozen=True)
class FromNumpy:
    name: str
    source: np.ndarray

    def execute(self, env: Env) -> None:
        if self.name in env:
            raise KeyError(f"FromNumpy: key {self.name!r} already in env")
        env[self.name] = _buffer_cls().from_numpy(self.source)


@dataclass(frozen=True)
class Download:
    """Copy a buffer back into ``env[into]``.  Without strides: a plain
    copy of ``shape`` elements.  With strides (element units): the buffer is
    read whole and gathered on the host through the view's strides
    (reference: program.py:73-114)."""

    name: str
    shape: tuple[int, ...]
    dtype: Any
    into: str
    row_stride: int | None = None
    col_stride: int | None = None

    def execute(self, env: Env) -> None:
        buf = env[self.name]
        if self.row_stride is None:
            env[self.into] = buf.numpy(self.shape, self.dtype)
            return
        item = np.dtype(self.dtype).itemsize
        flat = buf.numpy((buf.nbytes // item,), self.dtype)
        if len(self.shape) == 2:
            strides = (self.row_stride * item, (self.col_stride or 0) * item)
        elif len(self.shape) == 1:
            strides = (self.row_stride * item,)
        else:
            raise ValueError(f"Download with strides supports 1D/2D shapes only; got {self.shape}")
        view = np.lib.stride_tricks.as_strided(flat, shape=self.shape, strides=strides, writeable=False)
        env[self.into] = np.ascontiguousarray(view)


@dataclass(frozen=True)
class Fill:
    name: str
    byte_value: int = 0

    def execute(self, env: Env) -> None:
        env[self.name].fill(self.byte_value)


class Kernel:
    """A kernel as fragments + context.  ``source`` renders lazily (cached);
    ``handle`` compiles through hiprtc on first use (cached per process by
    the shim, keyed by the exact source text)."""

    def __init__(self, fragments: tuple[Any, ...], ctx: CodegenContext, compile_options: str = "") -> None:
        self.fragments = tuple(fragments)
        self.ctx = ctx
        self.compile_options = compile_options
        self._source: str | None = None
        self._handle: int | None = None
        self._dims_slot_index = ctx.dims_buffer_index if ctx.dims_buffer_index is not None else len(ctx.buffers)

    @property
    def source(self) -> str:
        if self._source is None:
            self._source = CodegenEngine().render(list(self.fragments), self.ctx)
        return self._source

    @property
    def function_name(self) -> str:
        return self.ctx.function_name

    @property
    def dims_slot_index(self) -> int:
        return self._dims_slot_index

    @property
    def dim_names(self) -> tuple[str, ...]:
        return self.ctx.dims

    @property
    def workspace_bytes(self) -> int:
        """Device workspace the kernel takes as its last parameter (0: none)."""
        return self.ctx.workspace_bytes

    @property
    def handle(self) -> int:
        if self._handle is None:
            from metellus_amd.runtime import hip_backend

            self._handle = hip_backend.compile_kernel(self.source, self.function_name, self.compile_options)
        return self._handle

    def execute(self, env: Env) -> None:
        _ = self.source

    def batched(self) -> "Kernel":
        """The same kernel for a batch of identical programs: buffer
        parameters become per-program pointer tables indexed by blockIdx.z
        (launch with grid z = batch size)."""
        if self.ctx.batched:
            return self
        if self.ctx.workspace_bytes and not self.ctx.workspace_batched:
            raise ValueError(f"{self.function_name}: a kernel with a workspace (stream-K) is not batched")
        cached = getattr(self, "_batched", None)
        if cached is None:
            import dataclasses

            ctx = dataclasses.replace(self.ctx, batched=True, function_name=self.ctx.function_name + "_batched")
            cached = Kernel(self.fragments, ctx, self.compile_options)
            self._batched = cached
        return cached


@dataclass(frozen=True)
class Dispatch:
    """Launch ``kernel`` over ``grid`` workgroups of ``threads`` lanes.
    ``bindings`` name env Buffers in kernel-parameter order; ``dims`` are
    passed by value at ``kernel.dims_slot_index``.  With ``time_key`` the
    launch is event-timed and ``env[time_key]`` gets the kernel ms."""

    kernel: Kernel
    bindings: tuple[str, ...]
    dims: tuple[int, ...]
    grid: tuple[int, int, int]
    threads: tuple[int, int, int]
    time_key: str | None = None

    def execute(self, env: Env) -> None:
        if len(self.dims) != len(self.kernel.dim_names):
            raise ValueError(
                f"Dispatch: expected {len(self.kernel.dim_names)} dim values "
                f"({self.kernel.dim_names}), got {len(self.dims)}"
            )
        from metellus_amd.runtime import hip_backend

        slots = [env[name] for name in self.bindings]
        t = hip_backend.launch(
            self.kernel.handle,
            slots,
            self.dims,
            self.kernel.dims_slot_index,
            self.grid,
            self.threads,
            timed=self.time_key is not None,
            workspace=self.kernel.workspace_bytes,
        )
        if self.time_key is not None:
            env[self.time_key] = float(t)


@dataclass(frozen=True)
class Runtime:
    fragments: tuple[RuntimeFragment, ...] = field(default_factory=tuple)

    def run(self, env: Env | None = None) -> Env:
        if env is None:
            env = {}
        for step in self.fragments:
            step.execute(env)
        if any(isinstance(s, Dispatch) and s.kernel.workspace_bytes for s in self.fragments):
            from metellus_amd.runtime import hip_backend

            hip_backend.check_workspace()  # raises if a stream-K wait gave up
        return env

    def __add__(self, other: "Runtime") -> "Runtime":
        return Runtime(self.fragments + other.fragments)
