"""Turn assembled ``KernelGroup``s into an executable ``Runtime``
(reference: src/orchestrator/scheduler.py:59-221).

Plan, in order:

1. ``FromNumpy`` for every uploaded input (validated: every external input
   buffer has an upload and every upload is a program input);
2. ``Allocate`` for every non-input buffer, all of them before the first
   ``Dispatch`` and in first-use order (as the reference does), so the
   peak device footprint is the sum of the materialised buffers; each
   kernel is rendered here too, off the dispatch path;
3. one ``Dispatch`` per group; after it, every buffer whose last use it was
   is downloaded -- each view of it first (host gather through the view's
   strides), then the owner itself if it is a named tensor (which ends the
   buffer's life) -- or freed.

Fused intermediates never get a buffer, so they are never downloaded.
Frees are stream-ordered in the native shim, so they need no host sync.
"""

from __future__ import annotations

from collections.abc import Iterable

import numpy as np

from metellus_amd.orchestrator.builder import Operations
from metellus_amd.orchestrator.dag import build_dag
from metellus_amd.orchestrator.kernel_group import KernelGroup
from metellus_amd.runtime.program import Allocate, Dispatch, Download, Free, FromNumpy, Runtime


def schedule(
    ops: Operations,
    groups: tuple[KernelGroup, ...],
    *,
    profile: bool = False,
    outputs: Iterable[str] | None = None,
) -> Runtime:
    """``outputs`` (an extension; the reference always downloads every
    materialised tensor): download only these names and free every other
    buffer at its last use.  A name that no kernel materialises -- an
    intermediate fused into a kernel -- is an error."""
    program = ops.build()
    dag = build_dag(program)
    tensors = ops.tensors
    uploads = ops.uploads

    produced = {op.out.buffer_key for op in program}
    required = {tensors[n].buffer_key for n in dag.inputs} - produced
    provided = set(uploads)
    if required - provided:
        raise ValueError(f"schedule: input buffers {sorted(required - provided)} have no from_numpy upload")
    if provided - required:
        raise ValueError(f"schedule: uploads {sorted(provided - required)} do not correspond to any program input")

    nbytes = {op.out.buffer_key: op.out.nbytes for op in program}
    for name in uploads:
        nbytes[tensors[name].buffer_key] = tensors[name].nbytes
    input_keys = {tensors[n].buffer_key for n in uploads}

    live_keys = set(input_keys)
    for g in groups:
        live_keys.update(g.bindings)
    wanted: set[str] | None = None
    if outputs is not None:
        wanted = set(outputs)
        unknown = sorted(n for n in wanted if n not in tensors)
        if unknown:
            raise ValueError(f"schedule: unknown output names {unknown}")
        absent = sorted(n for n in wanted if n in uploads or tensors[n].buffer_key not in live_keys)
        if absent:
            raise ValueError(f"schedule: outputs {absent} are program inputs or not materialised by any kernel")
    names_by_key: dict[str, list[str]] = {}
    for name, t in tensors.items():
        if name not in uploads and t.buffer_key in live_keys and (wanted is None or name in wanted):
            names_by_key.setdefault(t.buffer_key, []).append(name)

    last_use: dict[str, int] = {}
    for i, g in enumerate(groups):
        for k in g.bindings:
            last_use[k] = i

    steps: list = [FromNumpy(name=tensors[n].buffer_key, source=arr) for n, arr in uploads.items()]
    allocated = set(input_keys)
    for g in groups:
        for k in g.bindings:
            if k not in allocated:
                steps.append(Allocate(name=k, nbytes=nbytes[k]))
                allocated.add(k)
        steps.append(g.kernel)

    retired: set[str] = set()
    for i, g in enumerate(groups):
        steps.append(
            Dispatch(
                kernel=g.kernel,
                bindings=g.bindings,
                dims=g.dims,
                grid=g.grid,
                threads=g.threads,
                time_key=f"t_{i}" if profile else None,
            )
        )
        for k in dict.fromkeys(g.bindings):  # unique, in binding order
            if k in retired or last_use.get(k) != i:
                continue
            names = names_by_key.get(k, [])
            for view in (n for n in names if n != k):
                t = tensors[view]
                steps.append(
                    Download(
                        name=t.buffer_key,
                        shape=t.shape,
                        dtype=np.float32,
                        into=t.name,
                        row_stride=t.row_stride,
                        col_stride=t.col_stride,
                    )
                )
            if k in names:
                t = tensors[k]
                steps.append(Download(name=k, shape=t.shape, dtype=np.float32, into=t.name))
            else:
                steps.append(Free(name=k))
            retired.add(k)
    return Runtime(tuple(steps))
