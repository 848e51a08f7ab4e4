"""Host-side pieces of bench.py: the size-sweep fit and the read-ceiling
kernel's launch contract (no GPU needed)."""

import pytest

import bench
from metellus_amd.runtime import hip_backend


def _records(rate_gbps, t0_us, sizes, config, kernel):
    return [{"config": config.format(s=s), "kernel": kernel, "work": float(b),
             "ms_mean": (t0_us * 1e-6 + b / (rate_gbps * 1e9)) * 1e3} for s, b in sizes]


def test_fit_sweep_recovers_rate_and_fixed_cost():
    sizes = [(1, 335544320), (2, 671088640), (4, 1342177280)]
    recs = _records(6900.0, 2.7, sizes, "sweep C2 x{s}", "elementwise_out_fused")
    recs += _records(7100.0, -1.9, [(s, 2 * b) for s, b in sizes], "sweep C3 x{s}", "elementwise_e_fused")
    recs += _records(7000.0, 1.5, sizes, "sweep read x{s} grid 8192", "read_ceiling")
    recs += _records(6800.0, 3.0, sizes, "sweep read x{s} grid 2048", "read_ceiling")
    fits = {f["family"]: f for f in bench.fit_sweep(recs)}
    assert set(fits) == {"sweep C2 / elementwise_out_fused", "sweep C3 / elementwise_e_fused",
                         "sweep read / read_ceiling grid 8192", "sweep read / read_ceiling grid 2048"}
    f = fits["sweep C2 / elementwise_out_fused"]
    assert f["steady_GBps"] == pytest.approx(6900.0, abs=0.1) and f["fixed_us"] == pytest.approx(2.7, abs=0.01)
    f = fits["sweep C3 / elementwise_e_fused"]
    assert f["steady_GBps"] == pytest.approx(7100.0, abs=0.1) and f["fixed_us"] == pytest.approx(-1.9, abs=0.01)
    assert fits["sweep read / read_ceiling grid 2048"]["steady_GBps"] == pytest.approx(6800.0, abs=0.1)
    # per-size fractions: bytes / time / 8 TB/s
    b, t = sizes[0][1], 2.7e-6 + sizes[0][1] / 6.9e12
    assert fits["sweep C2 / elementwise_out_fused"]["frac_per_size"][0] == pytest.approx(b / t / 8e12, abs=1e-4)


def test_read_ceiling_source_compiles_for_gfx950():
    assert hip_backend.compile_only(bench.READ_CEILING_SRC) > 0


class _FakeBuffer:
    def __init__(self, nbytes):
        self.nbytes = nbytes


@pytest.mark.parametrize("nbytes", [8192 * 8192 * 4 + 4, (32768 * 5 + 2048) * 16, 8192 * 8192 * 8])
def test_read_ceiling_rejects_sizes_its_grids_cannot_split(nbytes):
    """Not a multiple of 16 bytes, a float4 count the grids do not divide, or
    more bytes than the buffer holds: refused before anything launches."""
    with pytest.raises(ValueError, match="read_ceiling"):
        bench.read_ceiling(_FakeBuffer(8192 * 8192 * 4), nbytes, 1, None, "x")


def test_read_ceiling_grids_divide_the_sweep_sizes():
    for s in bench.SWEEP_SCALES:
        n4 = 8192 * s * 8192 * 4 // 16
        assert all(n4 % g == 0 and n4 // g >= 256 for g in bench.READ_CEILING_GRIDS)


def test_traffic_is_read_only_for_the_profiled_kernel(tmp_path, monkeypatch):
    """roofline.traffic comes from the committed PMC summary only when that
    summary's row was profiled from the same kernel source (its SHA-256
    prefix); a row from another version of the kernel gives None and names
    both hashes."""
    prof = tmp_path / "profiles"
    prof.mkdir()
    (prof / "p.txt").write_text(
        "# header\n"
        f"{'config':32s} {'kernel':30s} {'source':16s} {'algorithmic B':>14s} {'read B':>14s} {'written B':>12s}\n"
        f"{'C4 MLP literal':32s} {'matmul_out_fused':30s} {'0123456789abcdef'} {'(mfma)':>14s} {4507783624:14d} {67108864:12d}\n"
        f"{'C2 sigmoid chain 4096x4096':32s} {'elementwise_out_fused':30s} {'fedcba9876543210'} {335544320:14d} "
        f"{268383129:14d} {67108864:12d}      0.9998\n")
    monkeypatch.setattr(bench, "ROOT", str(tmp_path))
    hit = bench.read_profile_traffic("C4 MLP literal", "matmul_out_fused", "0123456789abcdef", name="p.txt")
    assert hit["traffic"] == 4507783624 + 67108864 and hit["source"]["matches"]
    assert hit["source"]["file"] == "profiles/p.txt"
    stale = bench.read_profile_traffic("C4 MLP literal", "matmul_out_fused", "00000000ffffffff", name="p.txt")
    assert stale["traffic"] is None and not stale["source"]["matches"]
    assert stale["source"]["profiled_source_sha16"] == "0123456789abcdef"
    hbm = bench.read_profile_traffic("C2 sigmoid chain 4096x4096", "elementwise_out_fused", "fedcba9876543210",
                                     name="p.txt")
    assert hbm["traffic"] == 268383129 + 67108864
    missing = bench.read_profile_traffic("C5", "matmul_S_fused", "0123456789abcdef", name="p.txt")
    assert missing["traffic"] is None and missing["source"]["profiled_source_sha16"] is None
    assert bench.source_sha16("abc") == bench.source_sha16("abc") != bench.source_sha16("abd")


def test_sensor_parsing_and_absence(tmp_path):
    """The current clock level of a pp_dpm_* table is the line marked '*';
    a machine without the GPU's sysfs files gives no sensor summary."""
    assert bench.GpuSensors._dpm_mhz("0: 500Mhz\n1: 2105Mhz *\n2: 2400Mhz\n") == 2105.0
    assert bench.GpuSensors._dpm_mhz("0: 2000Mhz *\n") == 2000.0
    with pytest.raises(ValueError):
        bench.GpuSensors._dpm_mhz("0: 500Mhz\n1: 2400Mhz\n")
    s = bench.GpuSensors("0000:ff:1f.7")
    with s:
        pass
    assert s.paths == {} and s.summary() is None
