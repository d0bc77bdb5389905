"""CPU checks of the general loop's LDS maps for the 192-wide and 8-wave
tiles and for its staged f32 epilogue (whole 32-row blocks, or 16-row
halves where a block does not fit the ring), and of the plan's tile
coverage.

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


# ---- the general loop's staged f32 epilogue (GemmTile F32_*, gemm_kernel) ----
def f32_stage_params(bm, bn, bk, gm, gn, stages):
    """GemmTile's f32 staging constants: row bytes, chunks per row, rows per
    256-byte period, XOR width, rows per 64-lane read, rows per LDS pass."""
    wtn = bn // gn
    nw = gm * gn
    rowb = wtn * 4
    cpr = wtn // 4
    rpp = 1 if rowb >= 256 else 256 // rowb
    xor = min(cpr, 16)
    rpi = 64 // cpr
    ring = stages * (bm + bn) * bk * 2
    br = 32 if nw * 32 * rowb <= ring else 16
    assert nw * br * rowb <= ring, "no staging region fits the ring"
    return rowb, cpr, rpp, xor, rpi, br


def f32_stage_maps(wtn, rowb, cpr, rpp, xor, rpi, br, local_rows=True):
    """Per pass h: {LDS byte address: (block row, logical 16-byte chunk)}
    written by the active lanes, and [(lane, address, (block row, chunk))]
    read back: restates the staged f32 epilogue of gemm_kernel."""
    tn, hb = wtn // 32, 32 // br
    nld = 32 // rpi
    passes = []
    for h in range(hb):
        written, writers = {}, []
        for lane in range(64):
            rw, khalf = lane % 32, lane // 32
            if rw // br != h:
                continue
            rl = rw % br if local_rows else rw
            for j in range(tn):
                for g in range(4):
                    c = 8 * j + 2 * g + khalf
                    addr = rl * rowb + (c ^ ((rl // rpp) % xor)) * 16
                    assert addr not in written
                    written[addr] = (rw, c)
                    writers.append((lane, j, g, addr))
        reads = []
        for t in range(h * nld // hb, (h + 1) * nld // hb):
            for lane in range(64):
                r = (t - h * nld // hb) * rpi + lane // cpr
                q = lane % cpr
                addr = r * rowb + (q ^ ((r // rpp) % xor)) * 16
                reads.append((lane, addr, (t * rpi + lane // cpr, q)))
        passes.append((written, writers, reads))
    return passes


# (block, wave grid, stages, rows per pass): the reference's 128x64 case on
# 4x1 waves takes 16-row passes (4 x 32 rows x 256 bytes > its 24 KiB ring),
# as does 256x128x32 on 4x2 waves (64 KiB > 48 KiB); the others whole blocks
F32_TILES = [((128, 64, 32), (4, 1), 2, 16), ((64, 128, 32), (1, 4), 2, 32),
             ((64, 64, 32), (1, 1), 2, 32), ((64, 64, 32), (2, 2), 2, 32),
             ((128, 128, 64), (2, 2), 2, 32), ((256, 128, 32), (4, 2), 2, 16),
             ((128, 64, 64), (4, 2), 3, 32)]


@pytest.mark.parametrize("tile", F32_TILES, ids=lambda t: f"{t[0]}_w{t[1]}_s{t[2]}_r{t[3]}")
def test_f32_staged_epilogue_map(tile):
    """Each pass writes its rows' chunks once, inside the region, and every
    read finds the block row and chunk it stores; one 16-lane LDS cycle of a
    write or a read touches 16 different 16-byte bank groups."""
    (bm, bn, bk), (gm, gn), stages, rows = tile
    rowb, cpr, rpp, xor, rpi, br = f32_stage_params(bm, bn, bk, gm, gn, stages)
    assert br == rows
    for written, writers, reads in f32_stage_maps(bn // gn, rowb, cpr, rpp, xor, rpi, br):
        assert sorted(written) == list(range(0, br * rowb, 16)), "pass region not covered once"
        for lane, addr, want in reads:
            assert written[addr] == want, (lane, addr)
        for j in range(bn // gn // 32):
            for g in range(4):
                addrs = [a for (l, jj, gg, a) in sorted(writers) if jj == j and gg == g]
                for c0 in range(0, len(addrs), 16):
                    assert _bank_conflict_ways(addrs[c0:c0 + 16], 16, 16) == 1
        by_t = {}
        for i, (lane, addr, _) in enumerate(reads):
            by_t.setdefault(i // 64, []).append(addr)
        for addrs in by_t.values():
            assert _bank_conflict_ways(addrs, 16, 16) == 1


def test_f32_staged_epilogue_half_needs_local_rows():
    """Planted mistake: addressing a 16-row pass by the block row (rw) instead
    of the row in the pass overruns the 16-row region."""
    rowb, cpr, rpp, xor, rpi, br = f32_stage_params(128, 64, 32, 4, 1, 2)
    written = f32_stage_maps(64, rowb, cpr, rpp, xor, rpi, br, local_rows=False)[1][0]
    assert max(written) >= br * rowb
