"""Direct-to-LDS operand tiles (``mt_tile_dma``, ``mt_dma_slot`` and
``mt_swz`` in metellus_amd/csrc/mt_device.h), checked on the host: the
device helpers are compiled into a host program with hipcc and enumerated.

Invariants:

* the loader's wave-loads cover every (row, logical 16-byte slot) of the
  tile exactly once, inside the tile, and every wave issues the same number;
* ``mt_swz`` depends on the row modulo 16 only (the MFMA reader computes it
  from ``lane % 32`` for rows at multiples of 16 plus the lane), and the
  reader finds logical slot L of row r at physical slot L ^ mt_swz(r),
  where the loader put it;
* the MFMA reads (``mt_mfma_tile`` with a swizzled A or an n-major B: lane l
  reads row l % 32, logical slot (l / 32) * TK / 8 + s0 / 4, 128 bits) are
  free of bank conflicts whether the LDS serves 8 lanes x 16 B (128 B) or
  16 lanes x 16 B (256 B) per cycle, and in gfx950's measured passes of a
  ds_read_b128 (4 passes of 16 lanes, each the 8-lane groups k and k ^ 3 of
  one half-wave); the same reads from an unswizzled dense tile do conflict
  (so the check has teeth).
"""

import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "metellus_amd", "csrc", "mt_device.h")

HARNESS = r"""
#include <hip/hip_runtime.h>
#include <cstdio>
#include <vector>
#include MT_HEADER

// physical 16-byte slot index (row * S + p) the MFMA reader uses for lane l
template <int S, bool SWZ>
static unsigned read_slot(unsigned row_base, unsigned l, unsigned s0) {
    constexpr unsigned TK = 4 * S, HALF = TK / 2;
    const unsigned li = l & 31u, lh = l >> 5;
    const unsigned logical = (lh * HALF + s0) / 4u;
    const unsigned m = SWZ ? mt_swz<S>(li) : 0u;  // what mt_mfma_tile computes
    return (row_base + li) * S + (logical ^ m);
}

// conflicts: lanes in groups of G (G = 8: 128 B/cycle; G = 16: 256 B/cycle)
// must hit pairwise distinct 16-byte bank groups (slot index mod G).
// G = 0: gfx950's measured passes of a ds_read_b128 -- 4 passes of 16 lanes,
// each the 8-lane groups k and k ^ 3 of one half-wave, 256 B of banks.
static unsigned hw_pass(unsigned l) { return 2u * (l >> 5) + (((l >> 3) ^ (l >> 4)) & 1u); }

template <int S, bool SWZ>
static int conflicts(unsigned G) {
    int bad = 0;
    constexpr unsigned HALF = 2 * S;
    for (unsigned base = 0; base < 64; base += 16)
        for (unsigned s0 = 0; s0 < HALF; s0 += 4) {
            if (G == 0) {
                for (unsigned p = 0; p < 4; ++p) {
                    std::vector<int> seen(16, 0);
                    for (unsigned l = 0; l < 64; ++l)
                        if (hw_pass(l) == p) seen[read_slot<S, SWZ>(base, l, s0) % 16u]++;
                    for (unsigned b = 0; b < 16; ++b) bad += seen[b] > 1;
                }
                continue;
            }
            for (unsigned g0 = 0; g0 < 64; g0 += G) {
                std::vector<int> seen(G, 0);
                for (unsigned l = g0; l < g0 + G; ++l) seen[read_slot<S, SWZ>(base, l, s0) % G]++;
                for (unsigned b = 0; b < G; ++b) bad += seen[b] > 1;
            }
        }
    return bad;
}

template <int ROWS, int COLS, int NT, bool SWZ>
static int check_tile() {
    using T = mt_tile_dma<ROWS, COLS, NT, SWZ>;
    constexpr int S = T::S;
    std::vector<int> cover(ROWS * S, 0);
    std::vector<int> phys_of(ROWS * S, -1);
    for (unsigned w = 0; w < NT / 64; ++w)
        for (int q = 0; q < T::PERW; ++q) {
            const unsigned inst = w * T::PERW + q;
            for (unsigned lane = 0; lane < 64; ++lane) {
                unsigned r, logical;
                mt_dma_slot<S, SWZ>(inst, lane, r, logical);
                if (r >= (unsigned)ROWS || logical >= (unsigned)S) { std::printf("FAIL out of tile %d %d\n", ROWS, COLS); return 1; }
                cover[r * S + logical]++;
                phys_of[r * S + logical] = (int)(inst * 64 + lane);
            }
        }
    for (int i = 0; i < ROWS * S; ++i)
        if (cover[i] != 1) { std::printf("FAIL coverage %d %d at %d\n", ROWS, COLS, i); return 1; }
    if constexpr (SWZ)
        for (unsigned r = 0; r < (unsigned)ROWS; ++r)
            for (unsigned L = 0; L < (unsigned)S; ++L)
                if (phys_of[r * S + L] != (int)(r * S + (L ^ mt_swz<S>(r % 16u)))) {
                    std::printf("FAIL reader/loader disagree %d %d r=%u L=%u\n", ROWS, COLS, r, L);
                    return 1;
                }
    return 0;
}

int main() {
    for (unsigned r = 0; r < 4096; ++r) {
        if (mt_swz<8>(r) != mt_swz<8>(r % 16u) || mt_swz<4>(r) != mt_swz<4>(r % 16u) || mt_swz<8>(r) > 7u || mt_swz<4>(r) > 3u) {
            std::printf("FAIL swz period %u\n", r);
            return 1;
        }
    }
    // tiles the assembler uses: A 256x32 / 128x32 / 64x32 / 32x32 and
    // 256x16 (k-chunks of 32 and 16), n-major B 256x32, dense B 32x256,
    // 32x128, 16x256, 32x64
    int f = 0;
    f |= check_tile<256, 32, 512, true>();
    f |= check_tile<128, 32, 512, true>();
    f |= check_tile<64, 32, 256, true>();
    f |= check_tile<32, 32, 64, true>();
    f |= check_tile<256, 16, 512, true>();
    f |= check_tile<128, 16, 256, true>();
    f |= check_tile<32, 256, 512, false>();
    f |= check_tile<32, 128, 512, false>();
    f |= check_tile<16, 256, 512, false>();
    f |= check_tile<32, 64, 256, false>();
    if (f) return 1;
    const int c8a = conflicts<8, true>(8), c8b = conflicts<8, true>(16), c8h = conflicts<8, true>(0);
    const int c4a = conflicts<4, true>(8), c4b = conflicts<4, true>(16), c4h = conflicts<4, true>(0);
    if (c8a || c8b || c4a || c4b || c8h || c4h) {
        std::printf("FAIL conflicts %d %d %d %d %d %d\n", c8a, c8b, c4a, c4b, c8h, c4h);
        return 1;
    }
    const int n8 = conflicts<8, false>(8), n4 = conflicts<4, false>(16);
    std::printf("OK unswizzled_conflicts=%d,%d\n", n8, n4);
    return 0;
}
"""


@pytest.fixture(scope="module")
def harness(tmp_path_factory):
    d = tmp_path_factory.mktemp("lds_swizzle")
    src = d / "harness.hip"
    src.write_text(HARNESS)
    exe = d / "harness"
    hipcc = "/opt/rocm/bin/hipcc" if os.path.exists("/opt/rocm/bin/hipcc") else "hipcc"
    cmd = [hipcc, "--offload-arch=gfx950", "-O1", "-std=c++17", f'-DMT_HEADER="{HEADER}"', str(src), "-o", str(exe)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        pytest.fail(f"hipcc failed:\n{proc.stderr[-4000:]}")
    return exe


def test_dma_tiles_and_swizzle(harness):
    proc = subprocess.run([str(harness)], capture_output=True, text=True, timeout=60)
    assert proc.returncode == 0, proc.stdout + proc.stderr
    assert proc.stdout.startswith("OK"), proc.stdout
    n8, n4 = (int(x) for x in proc.stdout.split("=")[1].split(","))
    assert n8 > 0 and n4 > 0  # dense rows without the swizzle conflict


def test_assembler_picks_dma_layouts():
    from metellus_amd.api import compile_program
    from tests import gpu_cases

    def by(ops, batch=1):
        return {g.kernel.function_name: g for g in compile_program(ops, batch=batch)}

    g = by(gpu_cases.plain_matmul(512, 512, 512))["matmul_C_fused"]
    assert "mt_tile_dma<" in g.kernel.source and "true, false>(" in g.kernel.source
    # K^T stored n-major; Q row-major
    g = by(gpu_cases.attention_head(256, 64))["matmul_S_fused"]
    assert g.kernel.source.count("mt_tile_dma<") == 2 and "true, true>(" in g.kernel.source
    # a prologue on A keeps A on the register path; B (V) still loads directly
    g = by(gpu_cases.attention_head(256, 64))["matmul_O_fused"]
    assert g.kernel.source.count("mt_tile_dma<") == 1 and "commit_apply<" in g.kernel.source
    # ragged shapes keep the bounds-checked register path
    g = by(gpu_cases.plain_matmul(100, 70, 130))["matmul_C_fused"]
    assert "mt_tile_dma<" not in g.kernel.source


def test_dma_offsets_stay_within_32_bits():
    """A direct-to-LDS loader keeps each lane's byte offset from the tile
    origin in 32 bits; a row stride that would overflow them keeps that
    operand on the register path."""
    from metellus_amd.compute.matmul.config import TileConfig
    from metellus_amd.memory.memory import dma_offsets_fit
    from metellus_amd.orchestrator.assembly.matmul import dma_layouts
    from metellus_amd.orchestrator.ir import Tensor

    assert dma_offsets_fit(256, 32, 4096) and dma_offsets_fit(256, 32, "4096")
    # farthest byte: ((rows - 1) * rs + cols) * 4 against 2^32
    edge = ((1 << 30) - 32) // 255
    assert dma_offsets_fit(256, 32, edge) and not dma_offsets_fit(256, 32, edge + 1)
    assert not dma_offsets_fit(32, 256, "K")  # a stride that is not a literal
    tile = TileConfig(256, 256, 32, 2, 8)
    near = Tensor("A", (256, 32), row_stride=4096)
    far = Tensor("A", (256, 32), row_stride=(edge + 4) // 4 * 4)
    b = Tensor("B", (32, 256))
    assert dma_layouts(tile, (near,), (b,), (None,), (None,), True).a_layout == "swz"
    assert dma_layouts(tile, (far,), (b,), (None,), (None,), True).a_layout == "pad"
    b_far = Tensor("B", (32, 256), row_stride=(1 << 32) // 31 // 4 * 4)
    assert dma_layouts(tile, (near,), (b_far,), (None,), (None,), True).b_layout == "pad"
