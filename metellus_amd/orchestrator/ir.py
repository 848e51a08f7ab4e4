"""Primitive IR: fp32 tensors of rank <= 2 and four op kinds.

Restates the reference IR (reference: src/orchestrator/ir.py:1-491) with the
same classes, fields, defaults and validation messages, so programs built
against the reference build here unchanged:

* ``Tensor`` -- an SSA value with explicit (row_stride, col_stride) and a
  ``buffer_key`` naming its storage owner.  Transposes and contiguous
  reshapes are *views*: new SSA names that share the owner's buffer.
* ``MatmulOp``, ``ElementwiseOp``, ``ReductionOp`` (last axis only) and
  ``ShapeOp`` (strided copy), each validating shapes in ``__post_init__``.
"""

from __future__ import annotations

from dataclasses import dataclass
from enum import Enum

from metellus_amd.compute.elementwise.elementwise import BroadcastSpec, elementwise_arity


class Layout(str, Enum):
    """Logical storage order of a 2-D tensor (reference: ir.py:26-33)."""

    ROW_MAJOR = "row_major"
    COL_MAJOR = "col_major"

    def __str__(self) -> str:
        return self.value


def _default_strides(shape: tuple[int, ...], layout: Layout) -> tuple[int, int]:
    """(row_stride, col_stride) of the dense layout (reference: ir.py:36-50).
    0-D -> (0, 0); 1-D -> (1, 0)."""
    rank = len(shape)
    if rank == 0:
        return (0, 0)
    if rank == 1:
        return (1, 0)
    if rank == 2:
        rows, cols = shape
        return (cols, 1) if layout is Layout.ROW_MAJOR else (1, rows)
    raise ValueError(f"v0 supports 0D/1D/2D tensors only; got shape {shape}")


def _count(shape: tuple[int, ...]) -> int:
    n = 1
    for d in shape:
        n *= d
    return n


@dataclass(frozen=True)
class Tensor:
    """SSA value.  ``offset(row, col) = row*row_stride + col*col_stride``.
    ``row_stride``/``col_stride`` of -1 and ``buffer_key`` of "" are
    sentinels filled in ``__post_init__`` (dense strides; own buffer)."""

    name: str
    shape: tuple[int, ...]
    dtype: str = "float32"
    layout: Layout = Layout.ROW_MAJOR
    row_stride: int = -1
    col_stride: int = -1
    buffer_key: str = ""

    def __post_init__(self) -> None:
        if any(d <= 0 for d in self.shape):
            raise ValueError(f"tensor dimensions must be positive; got shape {self.shape}")
        if self.row_stride == -1 or self.col_stride == -1:
            rs, cs = _default_strides(self.shape, self.layout)
            if self.row_stride == -1:
                object.__setattr__(self, "row_stride", rs)
            if self.col_stride == -1:
                object.__setattr__(self, "col_stride", cs)
        if not self.buffer_key:
            object.__setattr__(self, "buffer_key", self.name)

    @property
    def nbytes(self) -> int:
        return 4 * _count(self.shape)  # fp32 only

    @property
    def element_count(self) -> int:
        return _count(self.shape)

    def linear_step(self) -> int | None:
        """Step ``c`` such that row-major iteration visits offsets 0, c, 2c,
        ...; None when iteration is not uniformly stepped
        (reference: ir.py:106-144)."""
        if len(self.shape) == 0:
            return 1
        if len(self.shape) == 1:
            return self.row_stride
        rows, cols = self.shape
        if rows == 1:
            return self.col_stride
        if cols == 1:
            return self.row_stride
        return self.col_stride if self.row_stride == cols * self.col_stride else None

    def is_contiguous(self) -> bool:
        return self.linear_step() == 1

    def transpose(self, name: str) -> Tensor:
        """2-D transpose as a metadata swap sharing the buffer
        (reference: ir.py:154-174)."""
        if len(self.shape) != 2:
            raise ValueError(f"transpose is 2D-only in v0; got shape {self.shape}")
        rows, cols = self.shape
        flipped = Layout.COL_MAJOR if self.layout is Layout.ROW_MAJOR else Layout.ROW_MAJOR
        return Tensor(
            name=name,
            shape=(cols, rows),
            dtype=self.dtype,
            layout=flipped,
            row_stride=self.col_stride,
            col_stride=self.row_stride,
            buffer_key=self.buffer_key,
        )

    def can_reshape_as_view(self, new_shape: tuple[int, ...]) -> bool:
        """Same shape (always), or same element count at rank 1-2 over a
        linearly iterable source (reference: ir.py:176-200)."""
        target = tuple(new_shape)
        if target == self.shape:
            return True
        if not 1 <= len(target) <= 2:
            return False
        if _count(target) != self.element_count:
            return False
        return self.linear_step() is not None

    def reshape_view(self, new_shape: tuple[int, ...], name: str) -> Tensor:
        """Metadata-only reshape (reference: ir.py:202-246)."""
        if not self.can_reshape_as_view(new_shape):
            raise ValueError(
                f"cannot reshape {self.name!r} {self.shape} → {tuple(new_shape)} "
                "as a metadata swap: needs same shape OR a linearly-iterable "
                "source with matching element count (ranks 0D/1D/2D only)"
            )
        target = tuple(new_shape)
        if target == self.shape:
            return Tensor(
                name=name,
                shape=self.shape,
                dtype=self.dtype,
                layout=self.layout,
                row_stride=self.row_stride,
                col_stride=self.col_stride,
                buffer_key=self.buffer_key,
            )
        step = self.linear_step()
        assert step is not None
        rs, cs = (step, 0) if len(target) == 1 else (target[1] * step, step)
        return Tensor(
            name=name,
            shape=target,
            dtype=self.dtype,
            layout=Layout.ROW_MAJOR,
            row_stride=rs,
            col_stride=cs,
            buffer_key=self.buffer_key,
        )


@dataclass(frozen=True)
class Scalar:
    """Compile-time constant secondary operand, inlined as an fp32 literal."""

    value: float


OperandValue = Tensor | Scalar


def _broadcast_target(primary_shape: tuple[int, ...], mode: BroadcastSpec) -> tuple[int, ...]:
    if mode is BroadcastSpec.NONE:
        return primary_shape
    if len(primary_shape) != 2:
        raise ValueError(f"broadcast={mode!r} requires a 2D primary; got shape {primary_shape}")
    rows, cols = primary_shape
    if mode is BroadcastSpec.SCALAR:
        return (1, 1)
    if mode is BroadcastSpec.ROW:
        return (1, cols)
    return (rows, 1)


def _validate_operand(label: str, primary: Tensor, operand: OperandValue, mode: BroadcastSpec) -> None:
    """(reference: ir.py:276-308)"""
    if isinstance(operand, Scalar):
        if mode is not BroadcastSpec.NONE:
            raise ValueError(
                f"{label}_broadcast={mode!r} cannot be set for a Scalar "
                "operand — scalars are inlined, not broadcast"
            )
        return
    want = _broadcast_target(primary.shape, mode)
    if operand.shape == want:
        return
    if mode is BroadcastSpec.NONE:
        raise ValueError(
            f"{label}-operand shape {operand.shape} must match "
            f"primary {primary.shape} when {label}_broadcast=NONE"
        )
    raise ValueError(
        f"{label}-operand shape {operand.shape} incompatible "
        f"with {label}_broadcast={mode!r} (expected {want})"
    )


@dataclass(frozen=True)
class MatmulOp:
    """out = a @ b (reference: ir.py:311-348)."""

    out: Tensor
    a: Tensor
    b: Tensor

    def __post_init__(self) -> None:
        if len(self.a.shape) != 2 or len(self.b.shape) != 2:
            raise ValueError(f"matmul operands must be 2D; got a={self.a.shape}, b={self.b.shape}")
        if self.a.shape[1] != self.b.shape[0]:
            raise ValueError(f"matmul contraction-axis mismatch: a={self.a.shape}, b={self.b.shape}")
        want = (self.a.shape[0], self.b.shape[1])
        if self.out.shape != want:
            raise ValueError(f"matmul out shape {self.out.shape} does not match a @ b = {want}")
        if not (self.a.dtype == self.b.dtype == self.out.dtype):
            raise ValueError(
                f"matmul dtypes must match; got a={self.a.dtype}, b={self.b.dtype}, out={self.out.dtype}"
            )

    @property
    def inputs(self) -> tuple[Tensor, ...]:
        return (self.a, self.b)


@dataclass(frozen=True)
class ElementwiseOp:
    """Pointwise op; ``operands[0]`` is the primary Tensor, later operands may
    be Scalars (reference: ir.py:351-413)."""

    out: Tensor
    op: str
    operands: tuple[OperandValue, ...]
    y_broadcast: BroadcastSpec = BroadcastSpec.NONE
    cond_broadcast: BroadcastSpec = BroadcastSpec.NONE

    def __post_init__(self) -> None:
        arity = elementwise_arity(self.op)
        if len(self.operands) != arity:
            raise ValueError(
                f"elementwise {self.op!r} is arity-{arity}, got {len(self.operands)} operands"
            )
        primary = self.operands[0]
        if not isinstance(primary, Tensor):
            raise ValueError(
                f"elementwise {self.op!r}: operand[0] must be a Tensor; got {primary!r}. "
                "Scalars are only allowed as secondary operands."
            )
        if self.out.shape != primary.shape:
            raise ValueError(
                f"elementwise out shape {self.out.shape} must match primary operand shape {primary.shape}"
            )
        if arity >= 2:
            _validate_operand("y", primary, self.operands[1], self.y_broadcast)
        elif self.y_broadcast is not BroadcastSpec.NONE:
            raise ValueError(f"y_broadcast={self.y_broadcast!r} set on arity-1 op {self.op!r}")
        if arity == 3:
            _validate_operand("cond", primary, self.operands[2], self.cond_broadcast)
        elif self.cond_broadcast is not BroadcastSpec.NONE:
            raise ValueError(
                f"cond_broadcast={self.cond_broadcast!r} set on arity-{arity} op {self.op!r}"
            )

    @property
    def inputs(self) -> tuple[Tensor, ...]:
        return tuple(o for o in self.operands if isinstance(o, Tensor))


@dataclass(frozen=True)
class ReductionOp:
    """Last-axis reduction of a 2-D tensor to 1-D (reference: ir.py:416-449)."""

    out: Tensor
    op: str
    input: Tensor
    axis: int = -1

    def __post_init__(self) -> None:
        if len(self.input.shape) != 2:
            raise ValueError(f"reduction input must be 2D in v0; got shape {self.input.shape}")
        axis = self.axis if self.axis >= 0 else len(self.input.shape) + self.axis
        if axis != len(self.input.shape) - 1:
            raise ValueError(
                f"reduction supports last axis only in v0; got axis={self.axis} on shape {self.input.shape}"
            )
        want = self.input.shape[:axis] + self.input.shape[axis + 1 :]
        if self.out.shape != want:
            raise ValueError(
                f"reduction out shape {self.out.shape} does not match input {self.input.shape} "
                f"reduced along axis {self.axis} (expected {want})"
            )

    @property
    def inputs(self) -> tuple[Tensor, ...]:
        return (self.input,)


@dataclass(frozen=True)
class ShapeOp:
    """Strided gather into a fresh dense buffer (reference: ir.py:452-487)."""

    out: Tensor
    input: Tensor

    def __post_init__(self) -> None:
        if self.input.element_count != self.out.element_count:
            raise ValueError(
                f"shape op element-count mismatch: input {self.input.shape} "
                f"({self.input.element_count} elems) → out {self.out.shape} "
                f"({self.out.element_count} elems)"
            )
        if self.input.dtype != self.out.dtype:
            raise ValueError(f"shape op dtype mismatch: input {self.input.dtype!r} → out {self.out.dtype!r}")
        if self.out.buffer_key != self.out.name:
            raise ValueError(
                "shape op out must own its buffer (buffer_key == name); "
                f"got name={self.out.name!r}, buffer_key={self.out.buffer_key!r}"
            )

    @property
    def inputs(self) -> tuple[Tensor, ...]:
        return (self.input,)


Op = MatmulOp | ElementwiseOp | ReductionOp | ShapeOp
Program = list[Op]
