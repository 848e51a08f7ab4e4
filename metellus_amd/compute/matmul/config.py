"""gfx950 matmul tile policy.

Replaces the reference's Apple tile picker (reference:
src/compute/matmul/config.py:40-51: 32x32x16 .. 128x64x32 tiles, four
32-wide simdgroups).  Here a workgroup of ``sg_M x sg_N`` wave64s computes a
``tile_M x tile_N`` output tile with fp32 MFMA (32x32 blocks); each wave owns
a ``(tile_M/sg_M) x (tile_N/sg_N)`` sub-tile, i.e. ``WM x WN`` accumulator
blocks of 16 registers.  A and B k-chunks of ``tile_K`` are double-buffered
in LDS: dense, XOR-swizzled tiles filled by direct-to-LDS loads, or rows
padded by ``a_pad``/``b_pad`` floats when filled through registers (see
``TileConfig.a_layout`` / ``b_layout``).

``select_tile_config`` scores each candidate by tile area x resident waves per
SIMD x useful fraction x grid fill (``tile_score``) and takes the best; the
16-wave tiles are candidates only when the caller says the operands leave the
registers for them (``wide``).  Large problems then run as persistent
workgroups (``persistent_workgroups``) with a stream-K last round
(``uses_stream_k``).
"""

from __future__ import annotations

from dataclasses import dataclass

NUM_CUS = 256  # MI355X compute units (8 XCDs x 32)


@dataclass(frozen=True)
class TileConfig:
    tile_M: int
    tile_N: int
    tile_K: int
    sg_M: int  # waves along M
    sg_N: int  # waves along N
    a_pad: int = 4
    b_pad: int = 4
    stages: int = 2
    c_pad: int = 4  # row padding of an LDS C tile (MatmulAccumToTgFragment)
    # LDS layouts of the operand tiles.  "pad": rows padded by a_pad / b_pad,
    # filled from registers.  Filled by direct-to-LDS loads instead (dense
    # rows): A "swz" = [tile_M][tile_K] with XOR-swizzled 16-byte slots;
    # B "dense" = [tile_K][tile_N]; B "nswz" = n-major [tile_N][tile_K],
    # swizzled like A (a transposed view such as K^T, read along K).
    a_layout: str = "pad"
    b_layout: str = "pad"

    @property
    def num_threads(self) -> int:
        return 64 * self.sg_M * self.sg_N

    @property
    def tg_x(self) -> int:
        return self.num_threads

    @property
    def tg_y(self) -> int:
        return 1

    @property
    def wave_M(self) -> int:
        return self.tile_M // self.sg_M

    @property
    def wave_N(self) -> int:
        return self.tile_N // self.sg_N

    @property
    def WM(self) -> int:
        return self.wave_M // 32

    @property
    def WN(self) -> int:
        return self.wave_N // 32

    @property
    def lda(self) -> int:
        return self.tile_K if self.a_layout == "swz" else self.tile_K + self.a_pad

    @property
    def ldb(self) -> int:
        """Row pitch of the B tile: along N (k-major layouts) or along K
        (the n-major layout)."""
        if self.b_layout == "dense":
            return self.tile_N
        if self.b_layout == "nswz":
            return self.tile_K
        return self.tile_N + self.b_pad

    def a_tile_shape(self) -> tuple[int, ...]:
        return (self.stages, self.tile_M, self.lda)

    def b_tile_shape(self) -> tuple[int, ...]:
        if self.b_layout == "nswz":
            return (self.stages, self.tile_N, self.tile_K)
        return (self.stages, self.tile_K, self.ldb)

    def validate(self) -> None:
        if self.wave_M % 32 or self.wave_N % 32 or self.tile_M % self.sg_M or self.tile_N % self.sg_N:
            raise ValueError(f"wave tile must be a multiple of 32x32: {self}")
        if self.tile_K % 8:
            raise ValueError(f"tile_K must be a multiple of 8: {self}")
        if self.lda % 4:
            raise ValueError(f"A tile row pitch must be a multiple of 4 floats (128-bit reads): {self}")
        if self.num_threads > 1024:
            raise ValueError(f"at most 1024 lanes per workgroup: {self}")
        if self.a_layout not in ("pad", "swz") or self.b_layout not in ("pad", "dense", "nswz"):
            raise ValueError(f"unknown operand tile layout: {self}")
        if (self.a_layout == "swz" or self.b_layout == "nswz") and self.tile_K not in (16, 32):
            raise ValueError(f"swizzled tiles are defined for tile_K 16 and 32: {self}")


def ceil_div(a: int, b: int) -> int:
    return (a + b - 1) // b


def is_aligned_shape(M: int, K: int, N: int, config: TileConfig) -> bool:
    return M % config.tile_M == 0 and N % config.tile_N == 0 and K % config.tile_K == 0


def grid_for(M: int, N: int, config: TileConfig) -> tuple[int, int, int]:
    return (ceil_div(N, config.tile_N), ceil_div(M, config.tile_M), 1)


# Candidate tiles.  One accumulator set: wave tiles up to 128x64 (128 acc
# registers); two sets (multi-anchor): up to 64x64 per anchor.
SINGLE_ANCHOR_TILES = (
    TileConfig(256, 256, 32, 2, 4),
    TileConfig(256, 128, 32, 4, 2),
    TileConfig(128, 256, 32, 2, 4),
    TileConfig(256, 128, 32, 2, 2),
    TileConfig(128, 256, 32, 2, 2),
    TileConfig(128, 128, 32, 4, 2),
    TileConfig(128, 128, 32, 2, 2),
    TileConfig(128, 64, 32, 2, 2),
    TileConfig(64, 128, 32, 2, 2),
    TileConfig(64, 64, 32, 2, 2),
    TileConfig(32, 32, 32, 1, 1),
)

# 16-wave tiles (4 waves per SIMD): offered when the operand chunks leave the
# registers for it (no full-size gathered prologue operands) -- measured on
# MI355X with direct-to-LDS loads: 4096^3 977.7 -> 968.0 us (2x8 waves of
# 128x32), C4 X @ W1 2650 -> 2609 us, C5 S 287.2 -> 283.6 us, C5 P @ V
# 280.3 -> 274.2 us (256x128 as 4x4 waves of 64x32).  4x4 waves of 64x64 on
# 256x256 were slower than 2x8 (987 us).
WIDE_TILES = (
    TileConfig(256, 256, 32, 2, 8),
    TileConfig(256, 128, 32, 4, 4),
)

DUAL_ANCHOR_TILES = (
    TileConfig(256, 128, 32, 4, 2),
    TileConfig(128, 128, 32, 2, 2),
    TileConfig(128, 64, 32, 2, 2),
    TileConfig(64, 128, 32, 2, 2),
    TileConfig(64, 64, 32, 2, 2),
    TileConfig(32, 32, 32, 1, 1),
)

LDS_BYTES = 163_840
VGPRS_PER_LANE = 512  # unified VGPR+AGPR file per SIMD lane (gfx950)

FORCE_TILE: TileConfig | None = None  # tuning override (measurement scripts)


def _pow2_at_least(x: int) -> int:
    p = 32
    while p < x:
        p *= 2
    return p


def tile_lds_bytes(t: TileConfig, anchors: int = 1) -> int:
    return 4 * t.stages * (t.tile_M * t.lda + anchors * t.tile_K * t.ldb)


def estimated_vgprs(t: TileConfig, anchors: int = 1) -> int:
    """Accumulators + prefetch registers + ~48 for addressing/operands."""
    acc = 16 * t.WM * t.WN * anchors
    prefetch = (t.tile_M * t.tile_K + anchors * t.tile_K * t.tile_N) // t.num_threads
    return acc + prefetch + 48


def tile_score(t: TileConfig, M: int, N: int, anchors: int = 1, batch: int = 1) -> tuple[float, float]:
    """(score, waves per SIMD).  Score = tile area (operand reuse per byte
    loaded) x resident waves per SIMD (latency hiding, capped at 4; from the
    LDS and register limits and the number of workgroups available) x the
    fraction of the tile that is real output x how well the grid fills the
    256 CUs."""
    wgs = batch * ceil_div(M, t.tile_M) * ceil_div(N, t.tile_N)
    waves = t.sg_M * t.sg_N
    by_lds = LDS_BYTES // tile_lds_bytes(t, anchors)
    by_vgpr = max(1, (4 * (VGPRS_PER_LANE // estimated_vgprs(t, anchors))) // waves)
    per_cu = max(1, min(by_lds, by_vgpr, ceil_div(wgs, NUM_CUS)))
    wps = per_cu * waves / 4
    useful = (M * N) / (ceil_div(M, t.tile_M) * t.tile_M * ceil_div(N, t.tile_N) * t.tile_N)
    fill = min(1.0, wgs / NUM_CUS)
    return t.tile_M * t.tile_N * min(wps, 4.0) * useful * fill, wps


PERSISTENT = True  # tuning switch for the persistent tile loop
PERSISTENT_CAPACITY: int | None = None  # override of resident workgroups (tests)
# Split the last partial round of a persistent loop by k-chunks (stream-K)
# instead of leaving workgroups idle; single (unbatched) problems only, and
# at most STREAM_K_MAX_WORKGROUPS workgroups (the workspace head holds one
# flag word per workgroup and the error word: MT_WS_HEAD - 1 flags).
STREAM_K = True
STREAM_K_MAX_WORKGROUPS = 1023


def resident_workgroups(t: TileConfig, anchors: int = 1, extra_lds: int = 0) -> int:
    """Workgroups of tile ``t`` one compute unit holds at once, from the LDS
    size (operand tiles plus ``extra_lds`` bytes the kernel declares beside
    them) and the register estimate (4 SIMDs x 512 registers per lane)."""
    by_lds = LDS_BYTES // (tile_lds_bytes(t, anchors) + extra_lds)
    by_vgpr = (4 * (VGPRS_PER_LANE // estimated_vgprs(t, anchors))) // (t.sg_M * t.sg_N)
    return max(1, min(by_lds, by_vgpr))


def persistent_workgroups(M: int, N: int, t: TileConfig, batch: int = 1, anchors: int = 1) -> int | None:
    """Workgroups per problem for a persistent tile loop, or None when every
    tile of every problem gets a resident workgroup in one round anyway."""
    if not PERSISTENT or t.stages != 2:
        return None
    tiles = ceil_div(M, t.tile_M) * ceil_div(N, t.tile_N)
    capacity = PERSISTENT_CAPACITY or NUM_CUS * resident_workgroups(t, anchors)
    if tiles * batch <= capacity:
        return None
    return min(tiles, max(1, capacity // batch))


def uses_stream_k(M: int, K: int, N: int, t: TileConfig, workgroups: int | None, batch: int = 1) -> bool:
    """A persistent loop of ``workgroups`` whose tiles are not a whole
    number of rounds: the last round runs as stream-K -- when its k-chunks
    are at least as many as the workgroups, so every workgroup's range holds
    work and a split tile's contributors are the workgroups just below its
    owner (the kernel's fixup relies on that)."""
    if not STREAM_K or workgroups is None or batch != 1 or workgroups > STREAM_K_MAX_WORKGROUPS:
        return False
    rem = (ceil_div(M, t.tile_M) * ceil_div(N, t.tile_N)) % workgroups
    return rem != 0 and rem * ceil_div(K, t.tile_K) >= workgroups


def select_tile_config(
    M: int, K: int, N: int, anchors: int = 1, batch: int = 1, wide: bool = False
) -> TileConfig:
    """Highest ``tile_score``; ties go to more resident waves, then more
    workgroups.  ``batch``
    identical problems launched together (grid z) count toward filling the
    GPU.  Tiles wider than the (power-of-two rounded) output are skipped.
    ``wide`` adds the 16-wave tiles (single anchor only).
    Measured on MI355X: 256x256 for 4096^3 and the C4/C5 Q.K^T GEMMs
    (16 waves when wide, else 8); 256x128 as 16 waves (wide) or 128x128 as
    8 waves for the C5 P.V GEMM (N = 128, batched heads)."""
    if FORCE_TILE is not None:
        return FORCE_TILE
    pool = SINGLE_ANCHOR_TILES if anchors == 1 else DUAL_ANCHOR_TILES
    if wide and anchors == 1:
        pool = WIDE_TILES + pool
    cands = [t for t in pool if t.tile_M <= _pow2_at_least(M) and t.tile_N <= _pow2_at_least(N)]
    best = None
    best_key = None
    for i, t in enumerate(cands):
        score, wps = tile_score(t, M, N, anchors, batch)
        wgs = ceil_div(M, t.tile_M) * ceil_div(N, t.tile_N)
        key = (score, wps, wgs, -i)
        if best_key is None or key > best_key:
            best, best_key = t, key
    return best
