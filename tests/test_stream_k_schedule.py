"""The stream-K schedule of persistent matmuls (``mt_stream_k`` in
metellus_amd/csrc/mt_device.h), checked on the host: the device struct is
compiled into a host program with hipcc and enumerated for every workgroup
of many (tiles, chunks, workgroups) cases.

Invariants (what the kernel's correctness and progress rest on):

* every (tile, k-chunk) unit is processed by exactly one workgroup;
* data-parallel items are whole tiles below ``dp``; stream-K items lie in
  the last ``tiles - dp`` tiles;
* a contributor item (chunk range not starting at 0) is always a
  workgroup's first item, so one workspace slot per workgroup suffices;
* the owner of a split tile (range starting at chunk 0, ending early)
  visits, with the kernel's own loop bounds, exactly the workgroups holding
  the rest of the tile (``mt_stream_k::contributor``, the kernel's loop),
  each contiguous with the previous one, each with a
  lower index than the owner (dispatched before it), each a contributor for
  that tile; and every contributor is visited by exactly one owner;
* when the stream-K units are at least as many as the workgroups (the only
  case the kernels use), a split tile's contributors are the consecutive
  workgroups w-1, w-2, ... below its owner w.
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

static int fail(const char* what, unsigned tiles, unsigned chunks, unsigned P, unsigned w) {
    std::printf("FAIL %s tiles=%u chunks=%u P=%u w=%u\n", what, tiles, chunks, P, w);
    return 1;
}

static int check(unsigned tiles, unsigned chunks, unsigned P) {
    std::vector<int> cover((size_t)tiles * chunks, 0);
    std::vector<int> consumed(P, 0);
    std::vector<int> contributes(P, -1);  // tile of each workgroup's contribution
    std::vector<mt_stream_k> sk(P);
    for (unsigned w = 0; w < P; ++w) sk[w].init(tiles, chunks, P, w);
    for (unsigned w = 0; w < P; ++w) {
        const mt_stream_k& s = sk[w];
        for (unsigned it = 0; it < s.items(); ++it) {
            unsigned t, kb, ke;
            s.item(it, t, kb, ke);
            if (t >= tiles || kb >= ke || ke > chunks) return fail("item bounds", tiles, chunks, P, w);
            for (unsigned k = kb; k < ke; ++k) cover[(size_t)t * chunks + k] += 1;
            if (t < s.dp && (kb != 0 || ke != chunks)) return fail("split data-parallel tile", tiles, chunks, P, w);
            if (kb != 0) {
                if (it != 0) return fail("contributor item not first", tiles, chunks, P, w);
                contributes[w] = (int)t;
            }
            if (kb == 0 && ke != chunks) {
                // the kernel's owner loop
                const unsigned long long tend = (unsigned long long)(t - s.dp + 1u) * chunks;
                unsigned next = ke, prev = 0u;
                for (unsigned c = s.contributor(1u, tend); c != 0u; c = s.contributor(c + 1u, tend)) {
                    if (c > w) return fail("owner waits past workgroup 0", tiles, chunks, P, w);
                    // with at least one unit per range the contributors are the
                    // consecutive workgroups w-1, w-2, ... (the kernel's fixup loop)
                    if (s.U >= s.P && c != prev + 1u) return fail("contributors not consecutive", tiles, chunks, P, w);
                    prev = c;
                    const unsigned cw = w - c;
                    unsigned ct, ckb, cke;
                    if (sk[cw].items() == 0) return fail("contributor without items", tiles, chunks, P, w);
                    sk[cw].item(0, ct, ckb, cke);
                    if (ct != t || ckb != next || ckb == 0) return fail("contributor range", tiles, chunks, P, w);
                    next = cke;
                    consumed[cw] += 1;
                }
                if (next != chunks) return fail("owner does not cover its tile", tiles, chunks, P, w);
            }
        }
    }
    for (size_t u = 0; u < cover.size(); ++u)
        if (cover[u] != 1) return fail("unit not covered exactly once", tiles, chunks, P, (unsigned)u);
    for (unsigned w = 0; w < P; ++w) {
        if ((contributes[w] >= 0) != (consumed[w] == 1) || consumed[w] > 1)
            return fail("contribution not consumed exactly once", tiles, chunks, P, w);
    }
    return 0;
}

int main() {
    const unsigned T[] = {1, 2, 3, 5, 7, 8, 13, 16, 31, 64, 97, 255, 256, 257, 511, 688, 1376, 2049};
    const unsigned C[] = {1, 2, 3, 4, 7, 16, 31, 128, 344};
    const unsigned Pw[] = {1, 2, 3, 4, 7, 13, 32, 100, 256, 512};
    unsigned n = 0;
    for (unsigned tiles : T)
        for (unsigned chunks : C)
            for (unsigned P : Pw) {
                if (check(tiles, chunks, P)) return 1;
                ++n;
            }
    std::printf("OK %u cases\n", n);
    return 0;
}
"""


@pytest.fixture(scope="module")
def harness(tmp_path_factory):
    d = tmp_path_factory.mktemp("stream_k")
    src = d / "harness.hip"
    src.write_text(HARNESS)
    exe = d / "harness"
    hipcc = "/opt/rocm/bin/hipcc" if os.path.exists("/opt/rocm/bin/hipcc") else "hipcc"
    cmd = [hipcc, "--offload-arch=gfx950", "-O1", f'-DMT_HEADER="{HEADER}"', str(src), "-o", str(exe)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        pytest.fail(f"hipcc failed:\n{proc.stderr[-4000:]}")
    return exe


def test_stream_k_schedule_invariants(harness):
    proc = subprocess.run([str(harness)], capture_output=True, text=True, timeout=120)
    assert proc.returncode == 0, proc.stdout + proc.stderr
    assert proc.stdout.startswith("OK"), proc.stdout


def test_stream_k_only_for_partial_rounds():
    from metellus_amd.compute.matmul.config import TileConfig, uses_stream_k

    t = TileConfig(256, 256, 32, 2, 4)
    assert uses_stream_k(4096, 4096, 11008, t, 256)  # 688 tiles
    assert not uses_stream_k(4096, 4096, 4096, t, 256)  # 256 tiles: whole rounds
    assert not uses_stream_k(4096, 4096, 11008, t, None)  # not persistent
    assert not uses_stream_k(4096, 4096, 11008, t, 8, batch=32)  # batched programs keep whole tiles
    # 176 leftover tiles x 1 k-chunk < 256 workgroups: some ranges would be empty
    assert not uses_stream_k(4096, 32, 11008, t, 256)
    assert uses_stream_k(4096, 64, 11008, t, 256)  # 352 units
