"""Spread loads (``MatmulMainloopFragment.spread``): a matmul whose prologue
gathers full-size operands issues the next k-chunk's register-path loads in
parts at the hook points of the current chunk's MFMA sequence.  Checked on
the host: the part predicate ``mt_in_part`` (device library) gives every
slot to exactly one part, in order; the mainloop never asks for more parts
than the MFMA sequence has hook points; the generated kernels put the
register loads (and only them) in the hook, on both the plain and the
persistent / stream-K paths, and compile for gfx950.  Results are checked
on the GPU by the suites that run these kernels (C4 at full size, stream-K
with gathered prologues, the random-program suite)."""

import os
import subprocess

import pytest

from metellus_amd.api import compile_program
from metellus_amd.compute.matmul import config
from metellus_amd.compute.matmul.matmul import MatmulMainloopFragment
from metellus_amd.orchestrator.assembly import matmul as am
from metellus_amd.runtime import hip_backend
from tests import gpu_cases

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "metellus_amd", "csrc", "mt_device.h")

HARNESS = r"""
#include <hip/hip_runtime.h>
#include <cstdio>
#include MT_HEADER

int main() {
    for (int n = 1; n <= 64; ++n)
        for (int Q = 1; Q <= 16; ++Q) {
            int prev = 0;
            for (int i = 0; i < n; ++i) {
                int owners = 0, part = -1;
                for (int q = 0; q < Q; ++q)
                    if (mt_in_part(i, n, q, Q)) ++owners, part = q;
                if (owners != 1) { std::printf("FAIL slot %d of %d in %d parts of %d\n", i, n, owners, Q); return 1; }
                if (part < prev) { std::printf("FAIL parts out of order n=%d Q=%d\n", n, Q); return 1; }
                prev = part;
            }
            // the default (0, 1) is the whole tile
            for (int i = 0; i < n; ++i)
                if (!mt_in_part(i, n, 0, 1)) { std::printf("FAIL default part n=%d\n", n); return 1; }
        }
    std::printf("OK\n");
    return 0;
}
"""


def test_parts_partition_every_slot_in_order(tmp_path):
    src = tmp_path / "parts.hip"
    src.write_text(HARNESS)
    exe = tmp_path / "parts"
    hipcc = "/opt/rocm/bin/hipcc" if os.path.exists("/opt/rocm/bin/hipcc") else "hipcc"
    proc = subprocess.run([hipcc, "--offload-arch=gfx950", "-O1", f'-DMT_HEADER="{HEADER}"', str(src), "-o", str(exe)],
                          capture_output=True, text=True)
    assert proc.returncode == 0, proc.stderr[-4000:]
    run = subprocess.run([str(exe)], capture_output=True, text=True, timeout=60)
    assert run.returncode == 0 and run.stdout.startswith("OK"), run.stdout


@pytest.mark.parametrize("tile_k", [8, 16, 32])
def test_parts_never_exceed_hook_points(tile_k):
    # mt_mfma_tile calls the hook once per group of 4 k-steps: tile_K / 8 times
    frag = MatmulMainloopFragment(tile_K=tile_k, fragments=(), K_dim_var="K", spread=16)
    register_loader = type("L", (), {"is_dma": False})()
    assert frag._spread([register_loader]) == tile_k // 8
    assert frag._spread([type("D", (), {"is_dma": True})()]) == 0  # direct-to-LDS loads stay before the MFMAs


def _w3(groups):
    return next(g for g in groups if g.kernel.function_name == "matmul_out_fused")


def test_full_operand_prologue_spreads_its_register_loads():
    g = _w3(compile_program(gpu_cases.mlp_block(512, 256, 768)))
    body = g.kernel.source.split('extern "C"')[1]
    hook = body.split("const auto mt_hook = [&](int mt_q) {")[1].split("};")[0]
    assert f"if (mt_q >= {am.LOAD_SPREAD}) return;" in hook
    assert f"fetch_gather<false>(g_h1, " in hook and f"xg_A_tile, mt_q, {am.LOAD_SPREAD});" in hook
    assert "ld_B_tile.fetch(" not in hook  # the direct-to-LDS W3 chunk is issued before the MFMAs
    before = body.split("const auto mt_hook")[0].split("for (unsigned kt")[1]
    assert "ld_B_tile.fetch(g_W3, " in before
    assert ", mt_hook);" in body.split("mt_mfma_tile<")[1]
    assert hip_backend.compile_only(g.kernel.source) > 0


@pytest.mark.parametrize("stream_k", [False, True])
def test_spread_on_persistent_paths(stream_k, monkeypatch):
    monkeypatch.setattr(config, "PERSISTENT", True)
    monkeypatch.setattr(config, "PERSISTENT_CAPACITY", 3)
    monkeypatch.setattr(config, "STREAM_K", stream_k)
    g = _w3(compile_program(gpu_cases.mlp_block(512, 256, 1024)))
    body = g.kernel.source.split('extern "C"')[1]
    assert ("mt_sk.init(" in body) == stream_k
    hook = body.split("const auto mt_hook = [&](int mt_q) {")[1].split("};")[0]
    # the next item's first chunk is loaded in parts too
    assert "} else if (mt_has_next) {" in hook and hook.count(f"mt_q, {am.LOAD_SPREAD});") == 2
    assert hip_backend.compile_only(g.kernel.source) > 0


def test_dma_only_kernels_and_the_switch_keep_the_burst(monkeypatch):
    body = compile_program(gpu_cases.plain_matmul(512, 512, 512))[0].kernel.source.split('extern "C"')[1]
    assert "mt_hook" not in body
    monkeypatch.setattr(am, "LOAD_SPREAD", 0)
    body = _w3(compile_program(gpu_cases.mlp_block(512, 256, 768))).kernel.source.split('extern "C"')[1]
    assert "mt_hook" not in body and "fetch_gather<false>(g_h1, " in body
