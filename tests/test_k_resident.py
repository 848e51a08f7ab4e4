"""The K-resident row-wave matmul (``MatmulKResidentFragment``, ``mt_kr_*`` in
metellus_amd/csrc/mt_device.h) on the CPU: which matmuls take it
(``assembly.matmul.k_resident``), how their columns split over workgroups,
what the kernel renders, that every form compiles, and -- with the device
helpers compiled into a host program -- its LDS layout:

* the B loader's wave-loads cover every (row, logical 16-byte slot) of the
  [128][K] chunk exactly once, and every wave issues the same number;
* the reader (lane group g = l/16, lane column c = l%16; quad t, column half
  h, block jj: row 64h + 4c + jj, logical slot gK/16 + t) finds each value
  where the loader put it, and the 4 values of one 128-bit read are k =
  gK/4 + 4t .. + 3, so the steps of the 4 lane groups cover every k once;
* the column map (block 4h + jj, lane column c -> 64h + 4c + jj) covers the
  chunk's 128 columns once;
* those reads are free of bank conflicts in gfx950's passes (a
  ds_read_b128 is served as 4 passes of 16 lanes, each pass the 8-lane
  groups k and k ^ 3 of one half-wave, from 64 4-byte banks -- measured
  with rocprof's LDS bank-conflict counter on fixed lane/address patterns)
  and in passes of 8 consecutive lanes, and the same reads of an
  unswizzled chunk conflict (so the check has teeth).
"""

from __future__ import annotations

import os
import subprocess

import numpy as np
import pytest

from metellus_amd.api import compile_program
from metellus_amd.orchestrator import Operations
from metellus_amd.orchestrator.assembly import matmul as mm
from metellus_amd.runtime import hip_backend
from tests.gpu_cases import attention_head

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "metellus_amd", "csrc", "mt_device.h")

HARNESS = r"""
#include <hip/hip_runtime.h>
#include <cstdio>
#include <vector>
#include MT_HEADER

// gfx950's ds_read_b128 passes: lanes l, l' share a pass iff they are in
// the same half-wave and ((l >> 3) ^ (l >> 4)) & 1 agree (8-lane groups k
// and k ^ 3), measured with rocprof's bank-conflict counter.
static unsigned mt_lds_pass(unsigned l) { return 2u * (l >> 5) + (((l >> 3) ^ (l >> 4)) & 1u); }

template <int K>
static int check(bool swizzled, int& conflicts8, int& conflicts16, int& conflicts_hw) {
    constexpr unsigned S = K / 4, T = K / 16;
    using L = mt_kr_dma<K, 1024>;
    std::vector<int> cover(128 * S, 0), phys_of(128 * S, -1);
    for (unsigned w = 0; w < 16; ++w)
        for (int q = 0; q < L::PERW; ++q) {
            const unsigned inst = w * L::PERW + q;
            for (unsigned lane = 0; lane < 64; ++lane) {
                unsigned r, logical;
                mt_kr_slot<K>(inst, lane, r, logical);
                if (r >= 128 || logical >= S) { std::printf("FAIL out of chunk K=%d\n", K); return 1; }
                cover[r * S + logical]++;
                phys_of[r * S + logical] = (int)(inst * 64 + lane);
            }
        }
    for (unsigned i = 0; i < 128 * S; ++i)
        if (cover[i] != 1) { std::printf("FAIL coverage K=%d at %u\n", K, i); return 1; }
    std::vector<int> kseen(K, 0), colseen(128, 0);
    conflicts8 = conflicts16 = conflicts_hw = 0;
    for (unsigned t = 0; t < T; ++t)
        for (int h = 0; h < 2; ++h)
            for (unsigned jj = 0; jj < 4; ++jj) {
                std::vector<unsigned> slot(64);
                for (unsigned lane = 0; lane < 64; ++lane) {
                    const unsigned c = lane & 15u, g = lane >> 4;
                    const unsigned n = 64u * h + 4u * c + jj;
                    const unsigned logical = g * T + t;
                    const unsigned sw = swizzled ? mt_kr_swz<K>(4u * c) : 0u;  // what mt_kr_chunk computes
                    if (swizzled && (mt_kr_swz<K>(n) != sw)) { std::printf("FAIL swz row K=%d\n", K); return 1; }
                    const unsigned phys = n * S + (logical ^ sw);
                    if (swizzled && phys_of[n * S + logical] != (int)phys) {
                        std::printf("FAIL reader/loader disagree K=%d n=%u L=%u\n", K, n, logical);
                        return 1;
                    }
                    slot[lane] = phys;
                    if (swizzled && h == 0 && jj == 0 && c == 0)
                        for (unsigned ss = 0; ss < 4; ++ss) kseen[4 * logical + ss]++;  // k of step 4t + ss
                    if (swizzled && t == 0 && g == 0) colseen[n]++;
                }
                // the models: 8 consecutive lanes per cycle (128 B), 16
                // consecutive lanes (256 B), and gfx950's measured passes
                // (8-lane groups k and k ^ 3 of a half-wave, 256 B)
                for (unsigned G : {8u, 16u})
                    for (unsigned g0 = 0; g0 < 64; g0 += G) {
                        std::vector<int> seen(G, 0);
                        for (unsigned l = g0; l < g0 + G; ++l) seen[slot[l] % G]++;
                        for (unsigned b = 0; b < G; ++b) (G == 8 ? conflicts8 : conflicts16) += seen[b] > 1;
                    }
                for (unsigned pass = 0; pass < 4; ++pass) {
                    std::vector<int> seen(16, 0);
                    for (unsigned l = 0; l < 64; ++l)
                        if (mt_lds_pass(l) == pass) seen[slot[l] % 16u]++;
                    for (unsigned b = 0; b < 16; ++b) conflicts_hw += seen[b] > 1;
                }
            }
    if (swizzled) {
        for (int k = 0; k < K; ++k) if (kseen[k] != 1) { std::printf("FAIL k coverage K=%d k=%d\n", K, k); return 1; }
        for (int n = 0; n < 128; ++n) if (colseen[n] != 1) { std::printf("FAIL column map K=%d n=%d\n", K, n); return 1; }
    }
    return 0;
}

int main() {
    int a8, a16, ah, b8, b16, bh, u8, u16, uh, v8, v16, vh;
    if (check<128>(true, a8, a16, ah) || check<64>(true, b8, b16, bh)) return 1;
    if (ah || bh || a8 || b8) { std::printf("FAIL conflicts %d %d %d %d\n", ah, bh, a8, b8); return 1; }
    check<128>(false, u8, u16, uh);
    check<64>(false, v8, v16, vh);
    std::printf("OK unswizzled_conflicts=%d,%d\n", uh, vh);
    return 0;
}
"""


@pytest.fixture(scope="module")
def harness(tmp_path_factory):
    d = tmp_path_factory.mktemp("k_resident")
    src = d / "harness.hip"
    src.write_text(HARNESS)
    exe = d / "harness"
    hipcc = "/opt/rocm/bin/hipcc" if os.path.exists("/opt/rocm/bin/hipcc") else "hipcc"
    cmd = [hipcc, "--offload-arch=gfx950", "-O1", "-std=c++17", f'-DMT_HEADER="{HEADER}"', str(src), "-o", str(exe)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        pytest.fail(f"hipcc failed:\n{proc.stderr[-4000:]}")
    return exe


def test_lds_layout_and_lane_maps(harness):
    proc = subprocess.run([str(harness)], capture_output=True, text=True, timeout=60)
    assert proc.returncode == 0, proc.stdout + proc.stderr
    assert proc.stdout.startswith("OK"), proc.stdout
    unswizzled = [int(x) for x in proc.stdout.split("=")[1].split(",")]
    assert all(n > 0 for n in unswizzled)  # dense rows without the swizzle conflict in both models


def _body(g) -> str:
    return g.kernel.source.split('extern "C"')[-1]


def _program(M=512, K=128, N=1024, prologue="none", epilogue=False, b_view=True) -> Operations:
    rng = np.random.default_rng(7)
    ops = Operations()
    ops.from_numpy(rng.standard_normal((M, K)).astype(np.float32), "A")
    if b_view:  # B = Bs^T, read along K
        ops.from_numpy(rng.standard_normal((N, K)).astype(np.float32), "Bs")
        ops.transpose("Bs", out="B")
    else:
        ops.from_numpy(rng.standard_normal((K, N)).astype(np.float32), "B")
    a = "A"
    if prologue == "row divisor":
        ops.from_numpy((rng.random(M) + 1.0).astype(np.float32), "s")
        ops.reshape("s", (M, 1), out="sv")
        ops.elementwise("div", out="P", operands=("A", "sv"), y_broadcast="col")
        a = "P"
    elif prologue == "scalar":
        ops.elementwise("mul", out="P", operands=("A", 0.5))
        a = "P"
    elif prologue == "column scale":
        ops.from_numpy(rng.random(K).astype(np.float32), "w")
        ops.reshape("w", (1, K), out="wv")
        ops.elementwise("mul", out="P", operands=("A", "wv"), y_broadcast="row")
        a = "P"
    ops.matmul(a=a, b="B", out="Y")
    if epilogue:
        ops.elementwise("max", out="Z", operands=("Y", 0.0))
    return ops


def _matmul_group(ops, batch=1):
    return [g for g in compile_program(ops, batch=batch) if g.kernel is not None and "matmul" in g.kernel.function_name][-1]


def test_attention_scores_take_k_resident_rows():
    gs = compile_program(attention_head(2048, 128, heads=32), batch=32)
    s = gs[0]
    assert s.kernel.function_name == "matmul_S_fused"
    assert s.grid == (1, 8, 1) and s.threads == (1024, 1, 1) and s.bindings == ("Q", "K", "Ss")
    body = s.kernel.batched().source.split('extern "C"')[-1]
    assert "B_tile[2][128][128]" in body and "mt_kr_chunk<128>(" in body and "A_tile" not in body
    assert "mt_kr_dma<128, 1024> ld_B(128u" in body and "for (unsigned ch = 0; ch < 16u; ++ch)" in body
    # stores go out between MFMA groups: the previous chunk's right half after
    # every other group of this chunk's left half, this chunk's left half
    # after the first four groups of its right half; the last right half
    # after the loop
    loop = body.split("for (unsigned ch = 0;")[1]
    assert "if (q < 8 && q % 2 == 0) {" in loop and "mt_store_row(1, q / 2, col_base - 128u);" in loop
    assert "} else if (q >= 8 && q < 12) {" in loop and "mt_store_row(0, q - 8, col_base);" in loop
    assert loop.index("mt_kr_chunk<128>(mt_a, &B_tile[ch & 1u][0][0], lane, acc, mt_hook);") < loop.index(
        "__builtin_amdgcn_s_waitcnt(0);") < loop.index("__syncthreads();")
    assert "for (int i = 0; i < 4; ++i) mt_store_row(1, i, mt_n0 + 1920u);" in loop
    assert "mt_buffer_store4<16>(mt_o, mt_rs, mt_voff," in body
    assert hip_backend.compile_only(s.kernel.batched().source) > 0
    # P @ V keeps the row-owning waves (K = 2048)
    assert "mt_rw_chunk(" in _body(gs[4])


@pytest.mark.parametrize("prologue", ["none", "row divisor", "scalar"])
@pytest.mark.parametrize("epilogue", [False, True])
@pytest.mark.parametrize("K", [64, 128])
def test_forms_compile(prologue, epilogue, K):
    g = _matmul_group(_program(K=K, prologue=prologue, epilogue=epilogue))
    body = _body(g)
    assert f"mt_kr_chunk<{K}>(" in body and f"B_tile[2][128][{K}]" in body
    assert ("xg(mt_row, 0u)" in body) == (prologue == "row divisor")
    assert ("xt(mt_a[q][e], mt_row," in body) == (prologue == "scalar")
    assert hip_backend.compile_only(g.kernel.source) > 0


@pytest.mark.parametrize("case", [
    dict(K=256), dict(K=96), dict(K=32), dict(M=500), dict(N=1000), dict(N=384), dict(b_view=False),
    dict(prologue="column scale"),
])
def test_cases_that_keep_other_kernels(case):
    g = _matmul_group(_program(**case))
    assert "mt_kr_chunk<" not in _body(g)


def test_switch_off_keeps_the_lds_tiled_kernel(monkeypatch):
    monkeypatch.setattr(mm, "K_RESIDENT", False)
    g = _matmul_group(_program())
    assert "mt_kr_chunk<" not in _body(g) and "mt_mfma_tile" in _body(g)


@pytest.mark.parametrize("M,N,batch,chunks", [
    (2048, 2048, 32, 16),   # C5: 256 row blocks fill the chip, each walks all 16 chunks
    (2048, 2048, 1, 1),     # one head: 8 row blocks, the columns split 16 ways
    (2048, 2048, 4, 2),
    (4096, 4096, 1, 2),     # 16 row blocks x 16 column groups
    (512, 1024, 1, 1),
    (8192, 1024, 8, 8),
])
def test_column_split(M, N, batch, chunks):
    assert mm.k_resident_chunks(M, N, batch) == chunks
    groups = (N // 128) // chunks
    assert groups * chunks == N // 128
    assert groups * batch * (M // 256) >= min(mm.NUM_CUS, (N // 128) * batch * (M // 256))


def test_batch_keeps_the_kernel_family():
    """A batched program and the same program alone take the same kernel
    (so the same per-element sum order); only the column split differs."""
    one = compile_program(attention_head(2048, 128))[0]
    many = compile_program(attention_head(2048, 128, heads=32), batch=32)[0]
    assert "mt_kr_chunk<128>(" in _body(one) and one.grid == (16, 8, 1)
    assert many.grid == (1, 8, 1)
