"""``Operations``: name-keyed builder for the primitive IR.

Same surface as the reference builder (reference:
src/orchestrator/builder.py:50-342): ``input``, ``from_numpy``, ``matmul``,
``elementwise``, ``transpose``, ``reshape``, ``reduction``, ``build``,
``tensors``, ``uploads``.  Validation is delegated to the op dataclasses;
the builder resolves names, keeps SSA freshness and records host payloads.

    ops = Operations()
    ops.from_numpy(a, "a"); ops.from_numpy(b, "b")
    ops.matmul(a="a", b="b", out="c")
    ops.elementwise("max", out="y", operands=("c", 0.0))   # relu
    program = ops.build()
"""

from __future__ import annotations

import numpy as np

from metellus_amd.compute.elementwise.elementwise import BroadcastSpec
from metellus_amd.orchestrator.ir import (
    ElementwiseOp,
    Layout,
    MatmulOp,
    OperandValue,
    Program,
    ReductionOp,
    Scalar,
    ShapeOp,
    Tensor,
)


def _addressable_elements(t: Tensor) -> int:
    """Elements a strided tensor can touch: (rows-1)*rs + (cols-1)*cs + 1
    (reference: builder.py:335-342)."""
    rank = len(t.shape)
    if rank == 0:
        return 1
    if rank == 1:
        return (t.shape[0] - 1) * t.row_stride + 1
    rows, cols = t.shape
    return (rows - 1) * t.row_stride + (cols - 1) * t.col_stride + 1


class Operations:
    """Mutable program builder; ``build()`` returns a snapshot list."""

    def __init__(self, dtype: str = "float32") -> None:
        self._dtype = dtype
        self._tensors: dict[str, Tensor] = {}
        self._ops: Program = []
        self._uploads: dict[str, np.ndarray] = {}

    # -- registry ------------------------------------------------------------

    def input(
        self,
        name: str,
        shape: tuple[int, ...],
        layout: Layout = Layout.ROW_MAJOR,
        row_stride: int | None = None,
        col_stride: int | None = None,
    ) -> Tensor:
        """Declare a caller-supplied tensor.  Redeclaring with the same shape
        returns the existing tensor."""
        return self._declare(name, shape, layout=layout, row_stride=row_stride, col_stride=col_stride)

    def from_numpy(self, arr: np.ndarray, name: str) -> Tensor:
        """Declare ``name`` as an input and record ``arr`` for upload.  Only
        float32 arrays and storage owners (not views) are accepted
        (reference: builder.py:80-118)."""
        if arr.dtype != np.float32:
            raise ValueError(f"from_numpy: array dtype must be float32; got {arr.dtype}")
        t = self._declare(name, tuple(arr.shape))
        if t.buffer_key != name:
            raise ValueError(
                f"from_numpy: {name!r} is a view of {t.buffer_key!r}; only storage owners can be uploaded"
            )
        if tuple(arr.shape) != t.shape:
            raise ValueError(
                f"from_numpy: array shape {tuple(arr.shape)} does not match declared tensor shape {t.shape}"
            )
        need = _addressable_elements(t)
        if arr.size < need:
            raise ValueError(
                f"from_numpy: array with shape {tuple(arr.shape)} provides {arr.size} elements, "
                f"but tensor {name!r} with strides (row_stride={t.row_stride}, "
                f"col_stride={t.col_stride}) can address {need} elements"
            )
        self._uploads[name] = arr
        return t

    def _declare(
        self,
        name: str,
        shape: tuple[int, ...],
        *,
        layout: Layout = Layout.ROW_MAJOR,
        row_stride: int | None = None,
        col_stride: int | None = None,
    ) -> Tensor:
        shape = tuple(shape)
        known = self._tensors.get(name)
        if known is not None:
            if known.shape != shape:
                raise ValueError(
                    f"tensor {name!r} already declared with shape {known.shape}, "
                    f"cannot redeclare as {shape}"
                )
            return known
        t = Tensor(
            name=name,
            shape=shape,
            dtype=self._dtype,
            layout=layout,
            row_stride=-1 if row_stride is None else row_stride,
            col_stride=-1 if col_stride is None else col_stride,
        )
        self._tensors[name] = t
        return t

    def _lookup(self, name: str) -> Tensor:
        t = self._tensors.get(name)
        if t is None:
            raise ValueError(
                f"tensor {name!r} is not declared — call ops.input(...) first or use an op that produces it"
            )
        return t

    def _fresh(self, name: str, shape: tuple[int, ...]) -> Tensor:
        """Output tensor for a new op; registered only after the op
        validates, so a rejected op leaves no stray name."""
        if name in self._tensors:
            raise ValueError(f"output tensor {name!r} already defined; IR is SSA — pick a fresh name")
        return Tensor(name=name, shape=tuple(shape), dtype=self._dtype)

    def _emit(self, out: Tensor, op) -> Tensor:
        self._tensors[out.name] = out
        self._ops.append(op)
        return out

    # -- ops -----------------------------------------------------------------

    def matmul(self, a: str, b: str, out: str) -> Tensor:
        ta, tb = self._lookup(a), self._lookup(b)
        t_out = self._fresh(out, (ta.shape[0], tb.shape[-1]))
        return self._emit(t_out, MatmulOp(out=t_out, a=ta, b=tb))

    def elementwise(
        self,
        op: str,
        out: str,
        operands: tuple[str | int | float, ...],
        y_broadcast: BroadcastSpec | str = BroadcastSpec.NONE,
        cond_broadcast: BroadcastSpec | str = BroadcastSpec.NONE,
    ) -> Tensor:
        """Tensor names resolve to declared tensors; int/float literals
        become ``Scalar`` operands (``bool`` is rejected)."""
        y_bc = BroadcastSpec(y_broadcast)
        c_bc = BroadcastSpec(cond_broadcast)
        resolved: list[OperandValue] = []
        for o in operands:
            if isinstance(o, str):
                resolved.append(self._lookup(o))
            elif isinstance(o, (int, float)) and not isinstance(o, bool):
                resolved.append(Scalar(value=float(o)))
            else:
                raise ValueError(f"operand {o!r} must be a tensor name (str) or numeric literal (int/float)")
        if not resolved or not isinstance(resolved[0], Tensor):
            first = operands[0] if operands else None
            raise ValueError(
                f"elementwise {op!r}: operand[0] must be a tensor name; got {first!r}. "
                "Scalars are only allowed as secondary operands."
            )
        t_out = self._fresh(out, resolved[0].shape)
        node = ElementwiseOp(
            out=t_out, op=op, operands=tuple(resolved), y_broadcast=y_bc, cond_broadcast=c_bc
        )
        return self._emit(t_out, node)

    def transpose(self, name: str, out: str) -> Tensor:
        """Metadata-only transpose: a view sharing ``name``'s buffer."""
        src = self._lookup(name)
        if out in self._tensors:
            raise ValueError(f"view tensor {out!r} already declared; pick a fresh name")
        view = src.transpose(out)
        self._tensors[out] = view
        return view

    def reshape(self, name: str, new_shape: tuple[int, ...], out: str) -> Tensor:
        """View when the source iterates linearly (or the shape is
        unchanged); otherwise a ``ShapeOp`` copy into a fresh buffer
        (reference: builder.py:259-305)."""
        src = self._lookup(name)
        if out in self._tensors:
            raise ValueError(f"reshape output {out!r} already declared; pick a fresh name")
        target = tuple(new_shape)
        if src.can_reshape_as_view(target):
            view = src.reshape_view(target, out)
            self._tensors[out] = view
            return view
        if not 1 <= len(target) <= 2:
            raise ValueError(f"reshape target rank must be 1D or 2D in v0; got {target}")
        count = 1
        for d in target:
            count *= d
        if count != src.element_count:
            raise ValueError(
                f"reshape element-count mismatch: {src.shape} ({src.element_count}) → {target} ({count})"
            )
        t_out = self._fresh(out, target)
        return self._emit(t_out, ShapeOp(out=t_out, input=src))

    def reduction(self, op: str, out: str, x: str, axis: int = -1) -> Tensor:
        from metellus_amd.compute.reduction.reduction import REDUCTION_OPS

        if op not in REDUCTION_OPS:
            raise ValueError(f"reduction op {op!r} not in {REDUCTION_OPS}")
        tx = self._lookup(x)
        ax = axis if axis >= 0 else len(tx.shape) + axis
        if 0 <= ax < len(tx.shape):
            shape = tx.shape[:ax] + tx.shape[ax + 1 :]
        else:
            shape = tx.shape[:-1] or (1,)
        t_out = self._fresh(out, shape)
        return self._emit(t_out, ReductionOp(out=t_out, op=op, input=tx, axis=axis))

    # -- results -------------------------------------------------------------

    def build(self) -> Program:
        return list(self._ops)

    @property
    def tensors(self) -> dict[str, Tensor]:
        return dict(self._tensors)

    @property
    def uploads(self) -> dict[str, np.ndarray]:
        return dict(self._uploads)
