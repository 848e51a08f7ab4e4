"""Public API: build an ``Operations`` program and ``run`` it."""

from metellus_amd.api.run import RunResult, compile_program, run

__all__ = ["RunResult", "compile_program", "run"]
