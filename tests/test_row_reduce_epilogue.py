"""The matmul -> reduction epilogue extension (``fusion.MATMUL_REDUCTION_EPILOGUES``,
off by default), checked on the CPU: the partition it makes, the kernels it
generates, and the lane map of its in-wave row reduction (``mt_rr_row`` in
metellus_amd/csrc/mt_device.h, compiled into a host program with hipcc)
against an independent simulation of the exchange steps."""

from __future__ import annotations

import os
import subprocess

import numpy as np
import pytest

from metellus_amd.api import compile_program
from metellus_amd.orchestrator import Operations, fusion
from metellus_amd.orchestrator.kernel_group import FusionStrategy
from metellus_amd.runtime import hip_backend
from tests import gpu_cases

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "metellus_amd", "csrc", "mt_device.h")

MAP_HARNESS = r"""
#include <hip/hip_runtime.h>
#include <cstdio>
#include MT_HEADER
template <int WM>
static void dump() {
    for (unsigned lane = 0; lane < 64; ++lane)
        for (int k = 0; k < MT_RR_KEEP(WM); ++k) std::printf("%d %u %d %u\n", WM, lane, k, mt_rr_row<WM>(lane, k));
}
int main() { dump<1>(); dump<2>(); dump<4>(); return 0; }
"""


@pytest.fixture(scope="module")
def row_map(tmp_path_factory):
    d = tmp_path_factory.mktemp("row_reduce")
    src = d / "map.hip"
    src.write_text(MAP_HARNESS)
    exe = d / "map"
    hipcc = "/opt/rocm/bin/hipcc" if os.path.exists("/opt/rocm/bin/hipcc") else "hipcc"
    cmd = [hipcc, "--offload-arch=gfx950", "-O1", "-std=c++17", f'-DMT_HEADER="{HEADER}"', str(src), "-o", str(exe)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        pytest.fail(f"hipcc failed:\n{proc.stderr[-4000:]}")
    out = subprocess.run([str(exe)], capture_output=True, text=True, timeout=60, check=True).stdout
    table: dict[tuple[int, int, int], int] = {}
    for line in out.split("\n"):
        if line:
            wm, lane, k, row = (int(x) for x in line.split())
            table[(wm, lane, k)] = row
    return table


def _simulate(wm: int) -> list[list[set[tuple[int, int]]]]:
    """The exchange steps as specified: every lane starts with its 16 WM
    values (block i, register r: row 32 i + 8 (r >> 2) + 4 (lane >> 5) +
    (r & 3), column lane % 32); for lane bits 0 .. 4 a lane keeps the half of
    its list its bit selects and merges in the partner's copy of that half;
    a lane with one value merges the partner's.  Returns, per lane, the
    (row, column) elements merged into each kept value."""
    lanes = [
        [{(32 * i + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3), lane % 32)} for i in range(wm) for r in range(16)]
        for lane in range(64)
    ]
    for b in (0, 1, 2, 3, 4):
        m = 1 << b
        new = []
        for lane in range(64):
            mine, theirs = lanes[lane], lanes[lane ^ m]
            n = len(mine)
            if n > 1:
                h = n // 2
                sel = slice(h, n) if lane & m else slice(0, h)
                new.append([a | c for a, c in zip(mine[sel], theirs[sel])])
            else:
                new.append([mine[0] | theirs[0]])
        lanes = new
    return lanes


@pytest.mark.parametrize("wm", [1, 2, 4])
def test_row_map_matches_the_exchange_steps(wm, row_map):
    sim = _simulate(wm)
    keep = max(1, 16 * wm // 32)
    rows_seen = set()
    for lane in range(64):
        assert len(sim[lane]) == keep
        for k, elems in enumerate(sim[lane]):
            rows = {r for r, _ in elems}
            assert rows == {row_map[(wm, lane, k)]}, (lane, k)
            assert {c for _, c in elems} == set(range(32))  # the whole row of the wave's 32 columns
            rows_seen.add(next(iter(rows)))
    assert rows_seen == set(range(32 * wm))


def test_row_map_differs_from_a_planted_order(row_map):
    """The map depends on the order of the exchange steps: the simulation run
    high bit first gives another map for 4-block waves."""
    lanes = [
        [{(32 * i + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3), lane % 32)} for i in range(4) for r in range(16)]
        for lane in range(64)
    ]
    for b in (4, 3, 2, 1, 0):
        m = 1 << b
        lanes = [
            [a | c for a, c in zip(lanes[lane][(slice(len(lanes[lane]) // 2, None) if lane & m else
                                               slice(0, len(lanes[lane]) // 2))],
                                   lanes[lane ^ m][(slice(len(lanes[lane]) // 2, None) if lane & m else
                                                    slice(0, len(lanes[lane]) // 2))])]
            for lane in range(64)
        ]
    planted = {(lane, k): next(iter(lanes[lane][k]))[0] for lane in range(64) for k in range(2)}
    assert any(planted[(lane, k)] != row_map[(4, lane, k)] for lane in range(64) for k in range(2))


def _groups(ops, flag, monkeypatch, batch=1):
    monkeypatch.setattr(fusion, "MATMUL_REDUCTION_EPILOGUES", flag)
    return compile_program(ops, batch=batch)


def test_reference_partition_with_the_flag_off(monkeypatch):
    gs = _groups(gpu_cases.attention_head(512, 64), False, monkeypatch)
    assert [g.strategy for g in gs] == [
        FusionStrategy.MATMUL_EPILOGUE_REGISTER,
        FusionStrategy.STANDALONE_REDUCTION,
        FusionStrategy.ELEMENTWISE_CHAIN,
        FusionStrategy.STANDALONE_REDUCTION,
        FusionStrategy.ELEMENTWISE_PROLOGUE_MATMUL,
    ]


def test_attention_row_max_joins_the_k_resident_score_kernel(monkeypatch):
    """C5's S = Q @ K^T takes the K-resident row waves; with the extension
    its row max is computed there too: every workgroup walks whole rows
    (grid x = 1 for any batch size), lanes fold their columns in order and
    the 16 lanes of a row combine by an xor-butterfly -- no LDS, no
    workspace."""
    for batch in (32, 1):
        gs = _groups(gpu_cases.attention_head(2048, 128, heads=32), True, monkeypatch, batch=batch)
        assert [g.strategy for g in gs] == [
            FusionStrategy.MATMUL_REDUCTION_EPILOGUE,
            FusionStrategy.ELEMENTWISE_CHAIN,
            FusionStrategy.STANDALONE_REDUCTION,
            FusionStrategy.ELEMENTWISE_PROLOGUE_MATMUL,
        ]
        s = gs[0]
        assert [op.out.name for op in s.ops] == ["S", "Ss", "m1"] and s.bindings == ("Q", "K", "Ss", "m1")
        assert s.grid == (1, 8, 1) and s.kernel.workspace_bytes == 0
        src = s.kernel.batched().source if batch > 1 else s.kernel.source
        body = src.split('extern "C"')[-1]
        assert "mt_kr_chunk<128>(" in body and "for (unsigned ch = 0; ch < 16u; ++ch)" in body
        assert "mt_red[i] = mt_rr_op<1>(mt_red[i], mt_o[j]);" in body
        assert [f"mt_xor_lanes<{m}u>(mt_red[i])" in body for m in (1, 2, 4, 8)] == [True] * 4
        assert "row_red" not in body and "mt_rr_finish<" not in body
        assert hip_backend.compile_only(src) > 0


def test_attention_row_max_joins_the_lds_tiled_score_kernel(monkeypatch):
    from metellus_amd.orchestrator.assembly import matmul as mm

    monkeypatch.setattr(mm, "K_RESIDENT", False)
    gs = _groups(gpu_cases.attention_head(2048, 128, heads=32), True, monkeypatch, batch=32)
    assert [g.strategy for g in gs] == [
        FusionStrategy.MATMUL_REDUCTION_EPILOGUE,
        FusionStrategy.ELEMENTWISE_CHAIN,
        FusionStrategy.STANDALONE_REDUCTION,
        FusionStrategy.ELEMENTWISE_PROLOGUE_MATMUL,
    ]
    s = gs[0]
    assert [op.out.name for op in s.ops] == ["S", "Ss", "m1"] and s.bindings == ("Q", "K", "Ss", "m1")
    # 32 heads x 8 row blocks fill the 256 workgroups: each walks one row
    # block's 8 column tiles and finishes its rows itself, no workspace
    assert s.grid == (8, 1, 1) and s.kernel.workspace_bytes == 0
    src = s.kernel.batched().source
    assert "mt_wave_row_reduce<4, 1, 1>(acc, lane, mt_rr_keep);" in src
    assert "row_red[9][256]" in src and "mt_rr_run = mt_rr_first ? r : fmaxf(mt_rr_run, r);" in src
    assert "mt_rr_finish<" not in src.split('extern "C"')[-1]
    assert hip_backend.compile_only(src) > 0


def test_few_row_blocks_combine_across_workgroups(monkeypatch):
    """Two row blocks of four column tiles: every tile runs in its own
    workgroup and the row blocks are combined through the workspace (the
    LDS-tiled kernel; K-resident rows off)."""
    from metellus_amd.orchestrator.assembly import matmul as mm

    monkeypatch.setattr(mm, "K_RESIDENT", False)
    gs = _groups(gpu_cases.attention_head(512, 64), True, monkeypatch)
    s = gs[0]
    assert s.grid == (4, 2, 1)
    # 2 row blocks x 4 column tiles of 256 row values, after the 1024 flag words
    assert s.kernel.workspace_bytes == 4 * (1024 + 2 * 4 * 256)
    body = s.kernel.source.split('extern "C"')[-1]
    assert body.count("mt_rr_finish<1, 256u, 1024u>(") == 2  # the previous tile's, the last tile's
    # a tile as wide as the row: the row completes in its workgroup
    one = _groups(_matmul_then("sum", 512, 64, 128), True, monkeypatch)[0]
    assert one.kernel.workspace_bytes == 0 and "mt_rr_run" in one.kernel.source


def _matmul_then(op: str, M: int, K: int, N: int, scale: float | None = None) -> Operations:
    rng = np.random.default_rng(7)
    ops = Operations()
    ops.from_numpy(rng.standard_normal((M, K)).astype(np.float32), "A")
    ops.from_numpy(rng.standard_normal((K, N)).astype(np.float32), "B")
    ops.matmul(a="A", b="B", out="Y")
    y = "Y"
    if scale is not None:
        ops.elementwise("mul", out="Yc", operands=("Y", scale))
        y = "Yc"
    ops.reduction(op, out="r", x=y)
    ops.elementwise("add", out="z", operands=(y, 1.0))  # another reader of the matmul output
    return ops


@pytest.mark.parametrize("op", ["sum", "max", "min", "product"])
@pytest.mark.parametrize("shape", [(512, 64, 1024), (300, 70, 520)])
def test_every_row_reduction_compiles(op, shape, monkeypatch):
    gs = _groups(_matmul_then(op, *shape, scale=0.5), True, monkeypatch)
    assert gs[0].strategy is FusionStrategy.MATMUL_REDUCTION_EPILOGUE
    assert gs[0].bindings == ("A", "B", "Yc", "r")
    src = gs[0].kernel.source
    assert ("col < N ? mt_y" in src) == (shape == (300, 70, 520))  # bounds only for the ragged shape
    assert hip_backend.compile_only(src) > 0


def test_no_stream_k_with_the_reduction(monkeypatch):
    """A persistent schedule whose last round would be split by k-chunks
    keeps whole tiles when the epilogue reduces rows."""
    body = lambda g: g.kernel.source.split('extern "C"')[-1]
    off = _groups(_matmul_then("max", 4096, 4096, 11008), False, monkeypatch)
    on = _groups(_matmul_then("max", 4096, 4096, 11008), True, monkeypatch)
    assert "mt_sk_wait(" in body(off[0]) and "mt_sk_wait(" not in body(on[0])
    assert "mt_rr_finish<" in body(on[0]) and hip_backend.compile_only(on[0].kernel.source) > 0


@pytest.mark.parametrize(
    "case",
    [
        "reduction of an elementwise output",
        "matmul with a prologue",
        "epilogue reading a tensor",
        "reduction through a view",
    ],
)
def test_cases_that_do_not_fuse(case, monkeypatch):
    rng = np.random.default_rng(3)
    ops = Operations()
    for name, shape in (("A", (256, 64)), ("B", (64, 512)), ("bias", (256, 512))):
        ops.from_numpy(rng.standard_normal(shape).astype(np.float32), name)
    if case == "matmul with a prologue":
        ops.elementwise("exp", out="Ae", operands=("A",))
        ops.matmul(a="Ae", b="B", out="Y")
        ops.reduction("max", out="r", x="Y")
    elif case == "epilogue reading a tensor":
        ops.matmul(a="A", b="B", out="Y0")
        ops.elementwise("add", out="Y", operands=("Y0", "bias"))
        ops.reduction("max", out="r", x="Y")
    elif case == "reduction through a view":
        ops.matmul(a="A", b="B", out="Y")
        ops.reshape("Y", (512, 256), out="Yv")
        ops.reduction("max", out="r", x="Yv")
    else:
        ops.matmul(a="A", b="B", out="Y")
        ops.elementwise("exp", out="E", operands=("Y",))
        ops.elementwise("add", out="F", operands=("E", 1.0))
        ops.reduction("sum", out="r", x="F")
        ops.elementwise("mul", out="G", operands=("E", 2.0))
    on = _groups(ops, True, monkeypatch)
    off = _groups(ops, False, monkeypatch)
    assert all(g.strategy is not FusionStrategy.MATMUL_REDUCTION_EPILOGUE for g in on)
    assert [g.strategy for g in on] == [g.strategy for g in off]


def test_residency_counts_the_row_array(monkeypatch):
    """The row-reduction epilogue's LDS row array (``rr_lds_shape``) is part
    of what limits resident workgroups: the local form's persistent grid and
    its choice of form count it beside the operand tiles.  With an LDS size
    that holds two workgroups' operand tiles but not two row arrays as well,
    one workgroup is resident, and the choice of form follows."""
    from metellus_amd.compute.matmul import config as cfg
    from metellus_amd.compute.matmul.matmul import rr_lds_shape
    from metellus_amd.orchestrator.assembly import matmul as mm

    tile = cfg.select_tile_config(512, 256, 1024)  # 128 x 128 tiles
    rows, cols = rr_lds_shape(tile)
    tiles = cfg.tile_lds_bytes(tile)
    assert cfg.resident_workgroups(tile) == mm.rr_resident_workgroups(tile) == 2  # gfx950's 160 KiB
    monkeypatch.setattr(cfg, "LDS_BYTES", 2 * tiles + 4 * rows * cols - 4)
    assert cfg.resident_workgroups(tile) == 2 and mm.rr_resident_workgroups(tile) == 1
    # 256 row blocks of 128 x 128 tiles fill one round of one resident
    # workgroup per CU (local form) but not of two
    assert mm.rr_local(256 * 128, 4 * 128, tile)
    monkeypatch.setattr(cfg, "LDS_BYTES", 2 * (tiles + 4 * rows * cols))
    assert mm.rr_resident_workgroups(tile) == 2
    assert not mm.rr_local(256 * 128, 4 * 128, tile)
