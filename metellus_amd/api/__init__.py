"""Public API: build an ``Operations`` program and ``run`` it (or
``run_batch`` several identical programs with one launch per kernel)."""

from metellus_amd.api.run import BatchRunner, RunResult, compile_program, run, run_batch

__all__ = ["BatchRunner", "RunResult", "compile_program", "run", "run_batch"]
