"""Extra input buffers pulled in by fused chains (reference:
src/orchestrator/assembly/extras.py:1-41).

Every template starts from fixed base slots (its anchor inputs and the
output); chain operands that are neither computed inside the kernel nor a
base input become extra kernel parameters, deduplicated by storage owner
(``buffer_key``) in order of first appearance.  That order is the
reference's binding order, which callers rely on."""

from __future__ import annotations

from dataclasses import dataclass, field

from metellus_amd.orchestrator.ir import Tensor


from metellus_amd.compute.elementwise.chain import param_name  # noqa: E402


def input_param(buffer_key: str) -> str:
    return f"const float* __restrict__ {param_name(buffer_key)}"


def output_param(buffer_key: str) -> str:
    return f"float* __restrict__ {param_name(buffer_key)}"


@dataclass
class Extras:
    buffers: list[str] = field(default_factory=list)
    bindings: list[str] = field(default_factory=list)
    base_slots_by_key: dict[str, int] = field(default_factory=dict)

    def add_tensor(self, t: Tensor, base_slot: int) -> int:
        """Register ``t`` as an input; returns its parameter slot."""
        key = t.buffer_key
        if key in self.base_slots_by_key:
            return self.base_slots_by_key[key]
        if key in self.bindings:
            return base_slot + self.bindings.index(key)
        self.buffers.append(input_param(key))
        self.bindings.append(key)
        return base_slot + len(self.bindings) - 1
