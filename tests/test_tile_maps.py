"""CPU checks of the general loop's LDS maps for the 192-wide and 8-wave
tiles, and of the plan's tile coverage.

The kernel (csrc/kernels/gemm_gfx950_impl.h, GemmTile / gemm_kernel) fills
each operand's LDS stage in rounds of one 16-byte chunk per lane: round i of
thread t writes stage chunk q = i * NT + t. For 192-wide B (24 chunks per
384-byte row) a round ends inside a row, so the lane's row q // 24 and chunk
q % 24 differ per round; the chunk holds logical chunk
(q % 24) ^ 4 ((row / B_PP) % B_MAXPH) with B_PP = 256 / gcd(row bytes, 256)
and B_MAXPH the largest power of two dividing the 64-byte segments per row
(at most 4). An operand stage smaller than its rounds (8 waves on a 32-deep
k-tile) leaves whole waves idle in the last round. These tests restate that
index math and check it against the oracle's swizzle (the plan's #tb.shared
encoding) and the brute-force LDS bank model; the plan tests check that the
plan derives the same encoding and binds the new tiles.
"""
import math
import re

import pytest

import oracle
from mini_triton_nvgpu_v1_amd import configs

from test_oracle import _bank_conflict_ways
from test_plan import MAINLINE, matmul_module, tb_opt


def b_swizzle(bn):
    """(rows per phase, phases) of the B stage: the kernel's GemmTile::B_PP,
    B_MAXPH and the plan's deriveSwizzle on 64-byte units."""
    row_bytes = bn * 2
    segs = row_bytes // 64
    return 256 // math.gcd(row_bytes, 256), min(4, segs & -segs)


def b_stage_map(bn, bk, nt):
    """{physical chunk index in the stage: (k row, logical chunk)} written by
    the B load rounds, restating gemm_kernel's issue_load for B."""
    bnc = bn // 8
    pp, mp = b_swizzle(bn)
    stage = bk * bnc
    rounds = -(-stage // nt)
    held = {}
    for i in range(rounds):
        for t in range(nt):
            q = i * nt + t
            if q >= stage:  # an idle wave of the last round: scratch row
                assert (i * nt + (t // 64) * 64) >= stage  # whole waves idle
                continue
            row, pc = q // bnc, q % bnc
            lc = pc ^ (4 * ((row // pp) % mp))
            assert 0 <= lc < bnc
            assert q not in held
            held[q] = (row, lc)
    return held


@pytest.mark.parametrize("bk", [32, 64])
@pytest.mark.parametrize("nt", [64, 128, 256, 512])
@pytest.mark.parametrize("bn", [64, 128, 192, 256])
def test_b_stage_load_map_is_the_plan_encoding(bn, bk, nt):
    """Every chunk of the B stage is written once per k-tile, and physical
    chunk p of k row r holds the logical chunk the plan's encoding puts
    there: the oracle's swizzle of its first column is p's first column."""
    pp, mp = b_swizzle(bn)
    held = b_stage_map(bn, bk, nt)
    bnc = bn // 8
    assert sorted(held) == list(range(bk * bnc))
    for q, (row, lc) in held.items():
        assert q // bnc == row
        phys = oracle.swizzle_minor(row, 8 * lc, pp, mp, 32, bn)
        assert phys == 8 * (q % bnc)


def test_b_swizzle_parameters():
    # power-of-two rows keep the previous parameters; 384-byte rows sit 128
    # bytes apart in the 256-byte bank period, so 2 rows per phase, and 6
    # segments admit 2 phases (an XOR of 2 or 3 would leave the row)
    assert b_swizzle(64) == (2, 2)
    assert b_swizzle(128) == (1, 4)
    assert b_swizzle(256) == (1, 4)
    assert b_swizzle(192) == (2, 2)
    for row in range(64):
        perm = [oracle.swizzle_minor(row, c, 2, 2, 32, 192) for c in range(192)]
        assert sorted(perm) == list(range(192))


def tr_read_addrs(bn, n0, k0, half, pp, mp):
    """Byte addresses of one ds_read_b64_tr_b16 of the general loop's B
    fragment (32x32x16 layout): lane l reads k row k0 + 8 (l / 32) + (l % 16)
    / 4 + 4 half, columns n0 + 16 ((l / 16) % 2) + 4 (l % 4) .. +3."""
    addrs = []
    for lane in range(64):
        k = k0 + 8 * (lane // 32) + (lane % 16) // 4 + 4 * half
        n = n0 + 16 * ((lane // 16) % 2) + 4 * (lane % 4)
        addrs.append(k * bn * 2 + oracle.swizzle_minor(k, n, pp, mp, 32, bn) * 2)
    return addrs


@pytest.mark.parametrize("bn", [64, 128, 192, 256])
def test_b_fragment_reads_conflict_free(bn):
    """Every 32-column tile of the row, every k step and both halves: one
    pass over the banks per 32-lane cycle with the derived encoding."""
    pp, mp = b_swizzle(bn)
    for n0 in range(0, bn, 32):
        for k0 in range(0, 64, 16):
            for half in (0, 1):
                assert _bank_conflict_ways(tr_read_addrs(bn, n0, k0, half, pp, mp), 8, 32) == 1


def test_b_fragment_reads_192_need_two_rows_per_phase():
    """Planted mistake: the power-of-two rule (1 row per phase) on 384-byte
    rows leaves k rows 2 apart on the same banks, a 2-way conflict."""
    assert _bank_conflict_ways(tr_read_addrs(192, 0, 0, 0, 1, 2), 8, 32) == 2


def test_idle_waves_of_a_partial_round():
    """A stage of fewer chunks than its rounds cover is whole waves' rounds:
    the idle part of the last round is whole waves (the kernel sends them to
    its scratch row with one wave-uniform test)."""
    for bm, bk, nt in [(64, 32, 512), (128, 32, 512), (192, 32, 512), (64, 64, 512)]:
        stage = bm * bk // 8
        assert stage % 64 == 0
        rounds = -(-stage // nt)
        live = {(i, w) for i in range(rounds) for w in range(nt // 64)
                if (i * nt + 64 * w) < stage}
        assert 64 * len(live) == stage


def test_plan_encodes_192_wide_b():
    """The plan derives the 384-byte-row B encoding (2 rows per phase, 2
    phases) and lowers a 128x192 tile to a compiled instance."""
    text = tb_opt(matmul_module(M=256, N=384, K=128, bm=128, bn=192, bk=64, warps=4,
                                stages=3), f"--pass-pipeline={MAINLINE}").stdout
    # the B stage ring buffer: memdesc [stages, block_k, block_n]
    b_ring = re.search(r"shape = \[3, 64, 192\], elementType = f16, "
                       r"encoding = #tb\.shared<([^>]*)>", text)
    assert b_ring, "no B stage buffer in the sealed module"
    assert "perPhase = 2, maxPhase = 2" in b_ring.group(1)
    assert "swizzlingByteWidth = 64" in b_ring.group(1)
    lowered = tb_opt(matmul_module(M=256, N=384, K=128, bm=128, bn=192, bk=64, warps=4,
                                   stages=3), "--pass-pipeline=builtin.module("
                     "tb-stage1-full-to-gfx950-pipeline{cubin-chip=gfx950})").stdout
    assert "tb_gemm_gfx950_128x192x64_w2x2_s3_out0" in lowered


# Tiles the reference's KernelConfig accepts (lib/Analysis/KernelConfig.cpp:
# 202-246) that no gfx950 kernel can hold: wave tiles of more than 256
# accumulator registers per lane, or more loads in flight per lane than the
# 6-bit vmcnt counts. Everything else in the sweep must bind.
def register_or_counter_infeasible(bm, bn, bk, nw, st):
    try:
        gm, gn = configs.wave_grid(bm, bn, nw)
    except ValueError:
        return "no wave grid of 32x32 tiles"
    if (bm // gm) * (bn // gn) > 256 * 64:
        return "accumulators"
    nt = 64 * nw
    lpt = -(-(bm * bk // 8) // nt) + -(-(bk * bn // 8) // nt)
    if (st - 1) * lpt > 63:
        return "vmcnt"
    if nw == 1 and bn == 256:
        return "one wave cannot load 256-wide B rows with one swizzle phase per lane"
    return None


def test_plan_binds_every_feasible_tile():
    """Sweep {64,128,192,256}^2 x block_k {32,64} x 1/2/4/8 waves x 2-4 stages
    (LDS ring within 160 KiB) through tb_plan_from_mlir: a configuration is
    refused only for a reason register_or_counter_infeasible names, or when
    every build of it spills (the plan's register truth)."""
    import mini_triton_nvgpu_v1_amd as tb
    bound, refused = 0, []
    for bm in (64, 128, 192, 256):
        for bn in (64, 128, 192, 256):
            for bk in (32, 64):
                for nw in (1, 2, 4, 8):
                    for st in (2, 3, 4):
                        if st * (bm + bn) * bk * 2 > 160 * 1024:
                            continue
                        w = configs.Workload("sweep", bm * 3, bn * 2, bk * 4, 1, 0,
                                             (bm, bn, bk), num_waves=nw, stages=st)
                        try:
                            tb.plan_from_mlir(w.mlir())
                            bound += 1
                        except tb.TbError as e:
                            why = register_or_counter_infeasible(bm, bn, bk, nw, st)
                            if why is None and "spill" not in str(e):
                                refused.append(((bm, bn, bk, nw, st), str(e)[:120]))
    assert not refused, refused
    assert bound >= 200
