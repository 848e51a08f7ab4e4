"""The shim's on-disk code-object cache across processes: a second process
loads what the first compiled; an entry whose stored key differs from the
wanted one (a hash collision, or a file from another compiler) is a miss
and is recompiled, never launched."""

from __future__ import annotations

import json
import os
import subprocess
import sys

import pytest

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

# Compile and run a small chain in a fresh process; print the cache counters
# and whether the result matched the oracle.
_CHILD = r"""
import json, sys
import numpy as np
sys.path.insert(0, sys.argv[1])
from metellus_amd.api import run
from metellus_amd.orchestrator import Operations
from metellus_amd.runtime import hip_backend
from oracle.ir_eval import evaluate
rng = np.random.default_rng(5)
ops = Operations()
ops.from_numpy(rng.standard_normal((64, 96)).astype(np.float32), "a")
ops.from_numpy(rng.standard_normal((64, 96)).astype(np.float32), "b")
ops.elementwise("mul", out="t", operands=("a", "b"))
ops.elementwise("add", out="out", operands=("t", 1.5))
res = run(ops)
ok = bool(np.array_equal(res.env["out"], evaluate(ops)["out"]))
compiled, hits = hip_backend.cache_stats()
print(json.dumps({"compiled": compiled, "hits": hits, "ok": ok}))
"""


def _child(cache_dir: str) -> dict:
    env = dict(os.environ, MT_KERNEL_CACHE_DIR=cache_dir)
    env.pop("MT_KERNEL_CACHE", None)
    proc = subprocess.run(
        [sys.executable, "-c", _CHILD, ROOT], env=env, capture_output=True, text=True, timeout=110
    )
    assert proc.returncode == 0, proc.stderr[-2000:]
    return json.loads(proc.stdout.strip().splitlines()[-1])


def _rewrite_each(cache: str, edit) -> None:
    for name in os.listdir(cache):
        path = os.path.join(cache, name)
        with open(path, "rb") as f:
            blob = bytearray(f.read())
        klen = int.from_bytes(blob[:8], "little")
        assert 0 < klen < len(blob) - 8
        with open(path, "wb") as f:
            f.write(bytes(edit(blob, klen)))


def test_disk_cache_reused_and_checked(tmp_path):
    cache = str(tmp_path / "co")
    first = _child(cache)
    n = first["compiled"]
    assert n >= 1 and first["hits"] == 0 and first["ok"]
    assert len([f for f in os.listdir(cache) if f.endswith(".co")]) == n

    assert _child(cache) == {"compiled": 0, "hits": n, "ok": True}

    def flip_key_byte(blob, klen):  # same file name, different stored key
        blob[8] ^= 0x01
        return blob

    _rewrite_each(cache, flip_key_byte)
    assert _child(cache) == {"compiled": n, "hits": 0, "ok": True}

    _rewrite_each(cache, lambda blob, klen: blob[: 8 + klen])  # key but no code object
    assert _child(cache) == {"compiled": n, "hits": 0, "ok": True}
