"""Code-generation choices that the GPU timings depend on, checked on the
generated source (no GPU): where matmul prologues are applied, and how
batched kernels address their per-program buffers."""

import re

import pytest

import numpy as np

from metellus_amd.api import compile_program
from metellus_amd.orchestrator import Operations
from metellus_amd.runtime import hip_backend
from tests import gpu_cases


def _by_name(groups):
    return {g.kernel.function_name: g for g in groups}


def test_broadcast_only_prologue_gathers_and_applies_at_commit():
    # P = e / s1 (a per-row divisor) folded into the P @ V loads: s1 is loaded
    # with the tile, the (fast) division runs at commit; k-chunks stay 32 wide
    g = _by_name(compile_program(gpu_cases.attention_head(256, 64)))["matmul_O_fused"]
    src = g.kernel.source
    assert "mt_tile_colvec_g<" in src and "ld_A_tile.template fetch_gather<false>(" in src
    # the divisor is a gathered operand: the commit tests it once per wave and
    # then divides as x * 1/y without a branch per element
    assert "ld_A_tile.template commit_apply_fast<" in src
    assert "xq_A_tile, xp_A_tile);" in src and "mt_div_plain(e.v[0])" in src
    helpers = src.split('extern "C"')[0]
    assert "mt_div_fast(" in helpers.split("float prologue_a(")[-1].split("}")[0]
    assert "mt_div_rcp(" in helpers.split("float prologue_a_plain(")[-1].split("}")[0]
    assert "ld_B_tile.fetch(g_V, " in src  # no transform on V: loaded straight into LDS
    assert ", 32, " in src.split("mt_mfma_tile<")[-1].split(">")[0] + ", "


def test_elementwise_division_stays_ieee():
    g = compile_program(gpu_cases.softmax(32, 100))[-1]  # p = e / s1 as an elementwise kernel
    assert "mt_div_fast(" not in g.kernel.source.split('extern "C"')[1]
    assert "mt_div_fast(" not in "".join(g.kernel.ctx.helpers)


def _mfma_tile_k(body: str) -> int:
    return int(body.split("mt_mfma_tile<")[1].split(">")[0].split(",")[2])


def test_full_operand_prologue_gathers_with_the_tile(monkeypatch):
    # (h1 * s * h2) @ W3: s and h2 are full matrices, loaded with the A tile
    # and multiplied in when the chunk is committed.  W3 goes straight to LDS,
    # which leaves the registers for 32-wide k-chunks; with W3 loaded through
    # registers too, the chunks are 16 wide.
    from metellus_amd.orchestrator.assembly import matmul as am

    g = _by_name(compile_program(gpu_cases.mlp_block(128, 128, 384)))["matmul_out_fused"]
    body = g.kernel.source.split('extern "C"')[1]
    assert "mt_tile_colvec_g<" in body and ", 2> ld_A_tile;" in body
    assert "ld_A_tile.template fetch_gather<" in body and "ld_A_tile.template commit_apply<" in body
    assert "ld_B_tile.fetch(g_W3, " in body and _mfma_tile_k(body) == 32
    assert hip_backend.compile_only(g.kernel.source) > 0
    monkeypatch.setattr(am, "DMA_LOADS", False)
    g = _by_name(compile_program(gpu_cases.mlp_block(128, 128, 384)))["matmul_out_fused"]
    body = g.kernel.source.split('extern "C"')[1]
    assert "mt_tile_dma<" not in body and _mfma_tile_k(body) == 16
    assert hip_backend.compile_only(g.kernel.source) > 0


def test_gather_switch_off_restores_fetch_time_transform(monkeypatch):
    from metellus_amd.orchestrator.assembly import matmul as am

    monkeypatch.setattr(am, "GATHER_PROLOGUES", False)
    g = _by_name(compile_program(gpu_cases.mlp_block(128, 128, 384)))["matmul_out_fused"]
    body = g.kernel.source.split('extern "C"')[1]
    assert "fetch_gather" not in body and "ld_A_tile.template fetch<false>(" in body


def test_batched_tables_hold_global_pointers_and_compile():
    groups = compile_program(gpu_cases.attention_head(128, 64), batch=4)
    for g in groups:
        k = g.kernel.batched()
        body = k.source.split('extern "C"')[1]
        assert "MT_GLOBAL float* const* __restrict__ g_" in body
        assert "_tab[blockIdx.z];" in body
        assert hip_backend.compile_only(k.source) > 0


def test_persistent_loop_only_when_tiles_exceed_one_round(monkeypatch):
    from metellus_amd.compute.matmul import config

    gemm = compile_program(gpu_cases.plain_matmul(4096, 4096, 4096))[0]
    assert gemm.grid == (16, 16, 1)  # 256 tiles of 256x256: one per CU
    assert "mt_t += gridDim.x" not in gemm.kernel.source

    monkeypatch.setattr(config, "PERSISTENT_CAPACITY", 2)
    monkeypatch.setattr(config, "STREAM_K", False)
    g = compile_program(gpu_cases.plain_matmul(192, 96, 320))[0]
    assert g.grid == (2, 1, 1)
    src = g.kernel.source
    assert "for (unsigned mt_t = blockIdx.x; mt_t < mt_tiles; mt_t += gridDim.x) {" in src
    assert "} else if (mt_has_next) {" in src and "}  // persistent tile loop" in src
    assert g.kernel.workspace_bytes == 0 and "mt_ws" not in src.split('extern "C"')[1]
    assert hip_backend.compile_only(src) > 0


def test_stream_k_kernel_takes_the_workspace_last(monkeypatch):
    from metellus_amd.compute.matmul import config
    from metellus_amd.compute.matmul.matmul import stream_k_workspace_bytes

    # C4's X @ W1: 688 tiles of 256x256 on 256 resident workgroups
    g = compile_program(gpu_cases.mlp_block(4096, 4096, 11008))[0]
    assert g.grid == (256, 1, 1)
    assert g.kernel.workspace_bytes == stream_k_workspace_bytes(256, 256, 256)
    body = g.kernel.source.split('extern "C"')[1]
    assert "const mt_dims dims,\n    float* mt_ws\n)" in body
    assert "mt_sk.init(mt_tiles, mt_chunks, gridDim.x, blockIdx.x);" in body
    assert "mt_sk_signal(" in body and "mt_sk_wait(" in body
    assert hip_backend.compile_only(g.kernel.source) > 0
    with pytest.raises(ValueError, match="not batched"):
        g.kernel.batched()
    # whole rounds keep the plain loop; the switch turns stream-K off
    assert compile_program(gpu_cases.plain_matmul(4096, 4096, 4096))[0].kernel.workspace_bytes == 0
    monkeypatch.setattr(config, "STREAM_K", False)
    g = compile_program(gpu_cases.mlp_block(4096, 4096, 11008))[0]
    assert g.kernel.workspace_bytes == 0 and "mt_t += gridDim.x" in g.kernel.source


def test_persistent_batched_grid_splits_capacity_over_programs(monkeypatch):
    from metellus_amd.compute.matmul import config

    monkeypatch.setattr(config, "PERSISTENT_CAPACITY", 8)
    groups = compile_program(gpu_cases.attention_head(256, 64), batch=3)
    s_kernel = groups[0]  # S = Q @ K^T, 256 x 256 output per program
    assert s_kernel.grid == (8 // 3, 1, 1)  # 2 workgroups per program, 3 programs in grid z
    assert hip_backend.compile_only(s_kernel.kernel.batched().source) > 0


def test_persistent_switch_off_restores_classic_grid(monkeypatch):
    from metellus_amd.compute.matmul import config

    monkeypatch.setattr(config, "PERSISTENT_CAPACITY", 2)
    monkeypatch.setattr(config, "PERSISTENT", False)
    g = compile_program(gpu_cases.plain_matmul(192, 96, 320))[0]
    assert g.grid[2] == 1 and g.grid[0] * g.grid[1] > 2


WAIT_CASES = {
    "gemm": (lambda: gpu_cases.plain_matmul(512, 512, 512), None),
    "attention": (lambda: gpu_cases.attention_head(512, 128), None),
    "mlp": (lambda: gpu_cases.mlp_block(256, 256, 512), None),
    "gemm persistent": (lambda: gpu_cases.plain_matmul(1024, 256, 1024), (4, False, "mt_t += gridDim.x")),
    "gemm stream-K": (lambda: gpu_cases.plain_matmul(1024, 256, 1024), (5, True, "mt_sk.init(")),
    "mlp stream-K": (lambda: gpu_cases.mlp_block(512, 256, 1024), (3, True, "mt_sk.init(")),
    "diamond stream-K": (lambda: gpu_cases.mlp_block(512, 256, 640, diamond=True), (6, True, "mt_sk.init(")),
}


@pytest.mark.parametrize("name", sorted(WAIT_CASES))
def test_direct_to_lds_kernels_wait_for_every_memory_operation(name, monkeypatch):
    # A direct-to-LDS chunk shares the vector-memory counter with the
    # epilogue's stores and with ordinary loads, and they do not retire in
    # issue order, so the only safe wait before the barrier that publishes a
    # chunk is a full s_waitcnt(0): a partial count can pass with the chunk
    # still in flight (a vmcnt(8) that counted the K-resident kernel's A
    # loads, issued after its first B chunk, let some waves read that chunk
    # before it had landed: 32 wrong elements in one of C5's 32 heads).
    # Checked in every form a wait can take in the kernel's whole source
    # (the device library included): the builtin and inline asm.
    from metellus_amd.compute.matmul import config

    build, loop = WAIT_CASES[name]
    if loop is not None:
        capacity, stream_k, marker = loop
        monkeypatch.setattr(config, "PERSISTENT", True)
        monkeypatch.setattr(config, "PERSISTENT_CAPACITY", capacity)
        monkeypatch.setattr(config, "STREAM_K", stream_k)
    body = lambda g: g.kernel.source.split('extern "C"')[-1]
    dma = [g for g in compile_program(build()) if "mt_tile_dma<" in body(g) or "mt_kr_dma<" in body(g)]
    assert dma
    if name == "attention":  # Q @ K^T on K-resident rows, P @ V LDS-tiled
        assert sum("mt_kr_dma<" in body(g) for g in dma) == 1 and sum("mt_tile_dma<" in body(g) for g in dma) == 1
    if loop is not None:
        assert any(marker in g.kernel.source.split('extern "C"')[-1] for g in dma), name
    for g in dma:
        src = g.kernel.source
        builtin = re.findall(r"__builtin_amdgcn_s_waitcnt\(([^)]*)\)", src)
        assert builtin and all(w.strip() == "0" for w in builtin), (g.kernel.function_name, builtin)
        asm_text = " ".join(re.findall(r'asm\s*(?:volatile\s*)?\(\s*((?:"[^"]*"\s*)+)', src))
        asm_waits = re.findall(r"s_waitcnt[^\\\"]*", asm_text)
        assert all(re.fullmatch(r"s_waitcnt\s+(0|vmcnt\(0\)(\s+lgkmcnt\(0\))?)\s*", w) for w in asm_waits), (
            g.kernel.function_name, asm_waits)
        assert hip_backend.compile_only(src) > 0


def test_epilogue_and_merge_division_stay_ieee():
    # (A @ B) / d and a diamond merged by division produce the output: IEEE
    ops = gpu_cases.plain_matmul(256, 128, 256)
    ops.from_numpy(np.ones(256, np.float32), "d")
    ops.reshape("d", (256, 1), out="dc")
    ops.elementwise("div", out="Y", operands=("C", "dc"), y_broadcast="col")
    (g,) = compile_program(ops)
    assert "mt_div_fast(" not in "".join(g.kernel.ctx.helpers) and "/" in "".join(g.kernel.ctx.helpers)
    ops = Operations()
    for n, shape in (("X", (256, 128)), ("W1", (128, 256)), ("W2", (128, 256))):
        ops.input(n, shape)
    ops.matmul(a="X", b="W1", out="h1")
    ops.matmul(a="X", b="W2", out="h2")
    ops.elementwise("div", out="z", operands=("h1", "h2"))
    (g,) = compile_program(ops)
    assert g.kernel.function_name.startswith("multi_anchor")
    assert "mt_div_fast(" not in "".join(g.kernel.ctx.helpers)


def test_k_invariant_gathers_are_loaded_once_per_tile(monkeypatch):
    # P @ V with P = e / s1: s1 depends on the row only, so the A loader
    # gathers it with a tile's first chunk and keeps it for the later ones;
    # on the persistent path the next tile's first chunk gathers afresh
    from metellus_amd.compute.matmul import config

    g = _by_name(compile_program(gpu_cases.attention_head(512, 64)))["matmul_O_fused"]
    loop = g.kernel.source.split("for (unsigned kt = 0; kt < n_chunks; ++kt)")[1]
    assert "ld_A_tile.template fetch_keep<false>(g_e, " in loop and "fetch_gather" not in loop
    assert hip_backend.compile_only(g.kernel.source) > 0
    monkeypatch.setattr(config, "PERSISTENT", True)
    monkeypatch.setattr(config, "PERSISTENT_CAPACITY", 2)
    monkeypatch.setattr(config, "STREAM_K", False)
    g = _by_name(compile_program(gpu_cases.attention_head(512, 64)))["matmul_O_fused"]
    loop = g.kernel.source.split("for (unsigned kt = mt_kb; kt < mt_ke; ++kt)")[1]
    more, nxt = loop.split("} else if (mt_has_next) {")
    assert "fetch_keep<" in more and "fetch_gather<" in nxt.split("}")[0]
    assert hip_backend.compile_only(g.kernel.source) > 0
    # full-size gathered operands change with k: gathered with every chunk
    w3 = _by_name(compile_program(gpu_cases.mlp_block(256, 256, 512)))["matmul_out_fused"]
    assert "fetch_keep" not in w3.kernel.source.split('extern "C"')[1]


def test_plain_divisors_only_for_gathered_divisors():
    """The plain commit applies when every division of a prologue divides by
    a gathered operand (known before the element); not for recip, not for a
    divisor computed in the chain, not without fast division."""
    from metellus_amd.compute.elementwise.chain import ChainCode
    from metellus_amd.orchestrator.ir import ElementwiseOp, Scalar, Tensor

    x, d, t = Tensor("x", (8, 8)), Tensor("d", (8, 8)), Tensor("t", (8, 8))
    div = ElementwiseOp(out=Tensor("q", (8, 8)), op="div", operands=(x, d))
    assert ChainCode((div,), ("x",), "p", fast_div=True).plain_divisors() == [0]
    assert ChainCode((div,), ("x",), "p", fast_div=False).plain_divisors() is None
    rec = ElementwiseOp(out=Tensor("r", (8, 8)), op="recip", operands=(x,))
    assert ChainCode((rec,), ("x",), "p", fast_div=True).plain_divisors() is None
    tt = ElementwiseOp(out=t, op="add", operands=(x, Scalar(1.0)))
    inner = ElementwiseOp(out=Tensor("q2", (8, 8)), op="div", operands=(d, t))  # divides by a chain value
    assert ChainCode((tt, inner), ("x",), "p", fast_div=True).plain_divisors() is None
    mul = ElementwiseOp(out=Tensor("m", (8, 8)), op="mul", operands=(x, d))
    assert ChainCode((mul,), ("x",), "p", fast_div=True).plain_divisors() is None
    code = ChainCode((div,), ("x",), "p", fast_div=True)
    assert code.plain_predicate_lambda() == "[=](const mt_vals<1>& e) -> bool { return mt_div_plain(e.v[0]); }"
    assert "p_plain(" in code.helpers()[1] and "mt_div_rcp(" in code.helpers()[1]


def test_plain_divisor_split_is_workgroup_uniform(monkeypatch):
    """The LDS-tiled mainloop tests a tile's gathered divisors once and runs
    one of two k loops, each with a barrier per chunk.  The test is a per-wave
    ballot, so the choice goes through __syncthreads_and: every wave of the
    workgroup enters the same loop and meets the same barriers."""
    from metellus_amd.orchestrator.assembly import matmul as am

    monkeypatch.setattr(am, "ROW_WAVES", False)
    g = _by_name(compile_program(gpu_cases.attention_head(512, 256)))["matmul_O_fused"]
    body = g.kernel.source.split('extern "C"')[1]
    split = [ln.strip() for ln in body.splitlines() if "mt_plain =" in ln]
    assert split and all(s.startswith("const bool mt_plain = __syncthreads_and((") for s in split)
    assert all(s.endswith(") ? 1 : 0) != 0;") and "all_plain<" in s for s in split)
    assert "if (mt_plain) {" in body
    assert hip_backend.compile_only(g.kernel.source) > 0


def test_asm_stores_keep_their_data_registers():
    """A 128-bit store reads its data registers after it issues.  The
    compiler inserts the wait states for the stores it emits, but not for a
    store inside inline asm (nor, on MI355X, for a buffer store with an
    SGPR soffset: C5 S lost the first element of 16-32 stores a run to the
    next row's value written right behind them).  Every store the device
    library issues from inline asm is followed by its own s_nop."""
    from metellus_amd.compute.fragments import device_header

    src = device_header()
    stores = re.findall(r'asm volatile\(\s*"((?:global|buffer)_store[^"]*)"', src)
    assert len(stores) >= 3, stores
    assert all(st.endswith("\\n\\ts_nop 1") for st in stores), stores
