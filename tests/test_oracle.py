"""Pins the CPU oracle (oracle/oracle.c) before anything is checked against it.

Each oracle function is checked against something other than its own formula:
published known-answer vectors, numpy/library routines, brute force on tiny
inputs, closed forms and invariants (bijections, partitions), chosen so that
a dropped term, wrong index or transposed operand fails a test. A planted
mistake (in the oracle, on the CPU) shows the checks bite.
"""
import math

import numpy as np
import pytest

import oracle


# ---- SplitMix64 ------------------------------------------------------------
def test_splitmix64_known_answers():
    # Vigna's reference splitmix64.c: state 0 -> first output 0xE220A8397B1DCDAF
    assert oracle.splitmix64_at(0, 0) == 0xE220A8397B1DCDAF
    # state 1234567 (the widely quoted test vector of the same generator)
    assert [oracle.splitmix64_at(1234567, i) for i in range(5)] == [
        6457827717110365317, 3203168211198807973, 9817491932198370423,
        4593380528125082431, 16408922859458223821]


def test_splitmix64_counter_form_equals_sequential_stream():
    # The counter form must equal stepping the generator's state i+1 times.
    M64 = (1 << 64) - 1
    state = 0x5EED0004
    for i in range(200):
        state = (state + 0x9E3779B97F4A7C15) & M64
        z = state
        z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & M64
        z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & M64
        z ^= z >> 31
        assert oracle.splitmix64_at(0x5EED0004, i) == z


def test_uniform_closed_form_and_range():
    L = oracle.lib()
    xs = [L.tbo_uniform_at(0x5EED0001, i) for i in range(4096)]
    for i, v in enumerate(xs[:64]):
        top = oracle.splitmix64_at(0x5EED0001, i) >> 40
        assert v == top / 2.0 ** 23 - 1.0
    arr = np.array(xs)
    assert arr.min() >= -1.0 and arr.max() < 1.0
    assert abs(arr.mean()) < 0.05  # 4096 draws: sd of the mean ~ 0.009


def test_normal_moments():
    L = oracle.lib()
    z = np.array([L.tbo_normal_at(0x5EED0004, i) for i in range(40000)])
    assert abs(z.mean()) < 0.03     # sd of mean 0.005
    assert abs(z.var() - 1.0) < 0.05  # a missing sqrt(2) or 2*pi would fail
    assert abs((np.abs(z) < 1.0).mean() - 0.6827) < 0.01


# ---- f16 conversion ----------------------------------------------------------
def test_f64_to_f16_matches_numpy():
    rng = np.random.default_rng(1)
    xs = np.concatenate([
        rng.standard_normal(20000) * np.exp(rng.uniform(-40, 12, 20000)),
        [0.0, -0.0, 65504.0, 65519.99, 65520.0, 1e6, -1e6, 2.0 ** -24,
         2.0 ** -25, 2.0 ** -25 * (1 + 2 ** -40), 3 * 2.0 ** -26, 2.0 ** -14,
         2.0 ** -14 - 2.0 ** -25, 1 + 2 ** -11, 1 + 3 * 2 ** -11, np.inf,
         -np.inf, 5e-324]])
    with np.errstate(over="ignore"):
        want = xs.astype(np.float16).view(np.uint16)
    got = np.array([oracle.f64_to_f16_bits(float(x)) for x in xs], np.uint16)
    assert np.array_equal(got, want)
    assert oracle.f64_to_f16_bits(float("nan")) & 0x7c00 == 0x7c00


def test_f16_to_f64_exhaustive():
    bits = np.arange(65536, dtype=np.uint16)
    want = bits.view(np.float16).astype(np.float64)
    got = np.array([oracle.f16_bits_to_f64(int(b)) for b in bits])
    finite = np.isfinite(want)
    assert np.array_equal(got[finite], want[finite])
    assert np.array_equal(np.isnan(got), np.isnan(want))


def test_fill_layout_and_seed_split():
    A = oracle.fill_f16(3, 5, 77, oracle.UNIFORM)
    for r in range(3):
        for c in range(5):
            v = oracle.lib().tbo_uniform_at(77, r * 5 + c)
            assert A[r, c] == np.float16(v)
    A2, B2 = oracle.config_inputs(4, 6, 16, 0x5EED0004, oracle.NORMAL)
    assert A2.shape == (4, 16) and B2.shape == (16, 6)
    assert B2[0, 0] == np.float16(oracle.lib().tbo_normal_at(0x5EED0004 ^ 0xB, 0) / 4.0)


# ---- GEMM oracle -------------------------------------------------------------
@pytest.mark.parametrize("M,N,K", [(1, 1, 1), (7, 5, 3), (64, 64, 32),
                                   (96, 80, 32), (33, 513, 70)])
def test_gemm_f64_matches_numpy(M, N, K):
    rng = np.random.default_rng(M * 1000 + N)
    A = rng.uniform(-1, 1, (M, K)).astype(np.float16)
    B = rng.uniform(-1, 1, (K, N)).astype(np.float16)
    want = A.astype(np.float64) @ B.astype(np.float64)
    got = oracle.gemm_f64(A, B)
    assert np.allclose(got, want, rtol=0, atol=1e-12)


def test_gemm_f64_brute_force_tiny_with_init_and_rows():
    rng = np.random.default_rng(3)
    A = rng.uniform(-1, 1, (5, 4)).astype(np.float16)
    B = rng.uniform(-1, 1, (4, 3)).astype(np.float16)
    init = rng.uniform(-1, 1, (5, 3)).astype(np.float32)
    got = oracle.gemm_f64(A, B, init=init, row_begin=1, row_end=4)
    for i in range(1, 4):
        for j in range(3):
            s = float(init[i, j])
            for k in range(4):
                s += float(A[i, k]) * float(B[k, j])
            assert abs(got[i - 1, j] - s) < 1e-12


def test_gemm_f64_not_transposed():
    # A non-square, non-symmetric case where A@B != (B.T@A.T).T would be
    # indistinguishable is avoided: use a structured pair with a known answer.
    A = np.array([[1, 2], [3, 4], [5, 6]], np.float16)  # 3x2
    B = np.array([[1, 0, 2], [0, 1, 3]], np.float16)      # 2x3
    got = oracle.gemm_f64(A, B)
    assert got.tolist() == [[1, 2, 8], [3, 4, 18], [5, 6, 28]]


def test_check_tolerance_counts_planted_errors():
    ref = np.full((4, 8), 10.0)
    got = ref.astype(np.float32).copy()
    assert oracle.check_tolerance(got, ref)[0] == 0
    got[1, 2] += 0.10          # bound is 1e-2 * (10 + 1) = 0.11 -> passes
    assert oracle.check_tolerance(got, ref)[0] == 0
    got[2, 3] += 0.12          # over the bound
    got[3, 7] = np.nan         # NaN must count as a failure
    bad, err, worst = oracle.check_tolerance(got, ref)
    assert bad == 2 and worst in [(2, 3), (3, 7)]
    bad16 = oracle.check_tolerance(got.astype(np.float16), ref)[0]
    assert bad16 >= 1


def test_check_tolerance_row_sample_indexes_absolute_rows():
    rng = np.random.default_rng(5)
    A = rng.uniform(-1, 1, (12, 8)).astype(np.float16)
    B = rng.uniform(-1, 1, (8, 6)).astype(np.float16)
    full = (A.astype(np.float64) @ B.astype(np.float64)).astype(np.float32)
    ref = oracle.gemm_f64(A, B, row_begin=5, row_end=9)
    assert oracle.check_tolerance(full, ref, row_begin=5)[0] == 0
    planted = full.copy()
    planted[2, 1] += 5.0  # outside the sampled rows: not counted
    assert oracle.check_tolerance(planted, ref, row_begin=5)[0] == 0
    planted[7, 4] += 5.0  # inside: counted at its absolute position
    bad, _, worst = oracle.check_tolerance(planted, ref, row_begin=5)
    assert bad == 1 and worst == (7, 4)
    with pytest.raises(ValueError):
        oracle.check_tolerance(full[5:9], ref, row_begin=5)  # a slice is refused


def test_planted_oracle_mistake_is_caught():
    """A transposed-operand or dropped-term bug in the oracle fails the pin."""
    rng = np.random.default_rng(9)
    A = rng.uniform(-1, 1, (16, 16)).astype(np.float16)
    B = rng.uniform(-1, 1, (16, 16)).astype(np.float16)
    good = oracle.gemm_f64(A, B)
    transposed = oracle.gemm_f64(B.T.copy(), A.T.copy()).T  # (A@B) recomputed
    assert np.allclose(good, transposed)
    wrong = oracle.gemm_f64(A, B.T.copy())  # planted mistake: B transposed
    assert oracle.check_tolerance(wrong.astype(np.float32), good)[0] > 0
    dropped = oracle.gemm_f64(A[:, :15].copy(), B[:15].copy())  # planted: last k term lost
    assert oracle.check_tolerance(dropped.astype(np.float32), good, rtol=1e-6)[0] > 0


# ---- fused epilogue steps ----------------------------------------------------
def _epi(x, **kw):
    r = np.array(x, dtype=np.float64).reshape(1, -1).copy()
    return oracle.epilogue_f64(r, **kw)[0]


def test_epilogue_activations_match_torch_cpu():
    """GELU (tanh form) and SiLU against torch's own CPU implementations in
    f64, an independent code path; relu against the definition."""
    import torch
    x = np.linspace(-8.0, 8.0, 1601)
    t = torch.from_numpy(x)
    gelu = torch.nn.functional.gelu(t, approximate="tanh").numpy()
    silu = torch.nn.functional.silu(t).numpy()
    assert np.allclose(_epi(x, act=2), gelu, rtol=0, atol=1e-13)
    assert np.allclose(_epi(x, act=3), silu, rtol=0, atol=1e-13)
    assert np.array_equal(_epi(x, act=1), np.where(x > 0, x, 0.0))
    assert np.array_equal(_epi(x, act=0), x)


def test_epilogue_closed_forms_and_symmetry():
    """f(0) = 0; f(x) - f(-x) = x for GELU-tanh and SiLU (their gates g
    satisfy g(x) + g(-x) = 1); f(x) -> x for large x and -> 0 for very
    negative x. A sign error in a term breaks the symmetry."""
    x = np.linspace(0.01, 6.0, 300)
    for act in (2, 3):
        assert _epi([0.0], act=act)[0] == 0.0
        assert np.allclose(_epi(x, act=act) - _epi(-x, act=act), x, atol=1e-12)
        assert abs(_epi([40.0], act=act)[0] - 40.0) < 1e-12
        assert abs(_epi([-40.0], act=act)[0]) < 1e-12
    # known values (tanh-GELU at 1: 0.5 (1 + tanh(sqrt(2/pi) 1.044715)))
    assert abs(_epi([1.0], act=2)[0] - 0.8411919906082768) < 1e-12
    assert abs(_epi([1.0], act=3)[0] - 1.0 / (1.0 + math.exp(-1.0))) < 1e-15


def test_epilogue_order_bias_activation_clamp():
    """bias before the activation, clamp last: each order mistake (planted
    here by composing the steps differently) gives a different answer."""
    bias = np.array([0.5, -2.0, 1.0])
    x = np.array([-1.0, 1.5, -3.0])
    got = _epi(x, bias=bias, act=3, clamp_bits=3, lo=-0.2, hi=0.4)
    z = x + bias
    expect = np.clip(z / (1 + np.exp(-z)), -0.2, 0.4)
    assert np.allclose(got, expect, atol=1e-15)
    act_first = np.clip(x / (1 + np.exp(-x)) + bias, -0.2, 0.4)
    clamp_first = (lambda c: c / (1 + np.exp(-c)))(np.clip(z, -0.2, 0.4))
    assert not np.allclose(got, act_first) and not np.allclose(got, clamp_first)
    # one-sided clamps
    assert np.array_equal(_epi([-5.0, 5.0], clamp_bits=1, lo=-1.0), [-1.0, 5.0])
    assert np.array_equal(_epi([-5.0, 5.0], clamp_bits=2, hi=1.0), [-5.0, 1.0])


@pytest.mark.parametrize("M,N,K", [(1, 1, 1), (13, 37, 29), (130, 70, 300)])
def test_gemm_f32_baseline_matches_numpy(M, N, K):
    rng = np.random.default_rng(K)
    A = rng.standard_normal((M, K)).astype(np.float32)
    B = rng.standard_normal((K, N)).astype(np.float32)
    got = oracle.gemm_f32(A, B, threads=2)
    want = A.astype(np.float64) @ B.astype(np.float64)
    assert np.allclose(got, want, rtol=1e-4, atol=1e-3 * math.sqrt(K))


# ---- program mapping / split / swizzle index math ----------------------------
def test_tile_mapping_is_row_major():
    for pid in range(12):
        assert oracle.program_to_tile(oracle.MAP_TILE, pid, 3, 4) == (pid // 4, pid % 4, 0)


def test_grouped_mapping_known_answer_192x128_gm2():
    # examples/smoke_grouped_192x128x32.mlir: 64x64 tiles -> tilesM=3, tilesN=2
    got = [oracle.program_to_tile(oracle.MAP_GROUPED, p, 3, 2, 2)[:2] for p in range(6)]
    assert got == [(0, 0), (1, 0), (0, 1), (1, 1), (2, 0), (2, 1)]


@pytest.mark.parametrize("tm,tn,gm", [(16, 16, 8), (3, 2, 2), (7, 5, 3),
                                      (43, 64, 8), (1, 9, 8), (9, 1, 4)])
def test_grouped_mapping_is_bijection(tm, tn, gm):
    for kind in (oracle.MAP_GROUPED, oracle.MAP_PERSISTENT_GROUPED):
        seen = {oracle.program_to_tile(kind, p, tm, tn, gm)[:2] for p in range(tm * tn)}
        assert seen == {(m, n) for m in range(tm) for n in range(tn)}
    # within a full group, consecutive programs walk down M first
    if tm >= gm:
        col0 = [oracle.program_to_tile(oracle.MAP_GROUPED, p, tm, tn, gm) for p in range(gm)]
        assert [c[0] for c in col0] == list(range(gm)) and {c[1] for c in col0} == {0}


def test_split_k_mapping_bijection_and_known_answer():
    tm, tn, s = 4, 3, 8
    seen = {oracle.program_to_tile(oracle.MAP_SPLIT_K, p, tm, tn, 1, s) for p in range(tm * tn * s)}
    assert seen == {(m, n, q) for m in range(tm) for n in range(tn) for q in range(s)}
    # examples/smoke_splitk_64x64x64.mlir: one tile, split 2 -> parts 0, 1
    assert [oracle.program_to_tile(oracle.MAP_SPLIT_K, p, 1, 1, 1, 2) for p in range(2)] == [
        (0, 0, 0), (0, 0, 1)]
    assert oracle.program_to_tile(oracle.MAP_SPLIT_K, 17, 4, 3, 1, 8) == (0, 2, 1)


@pytest.mark.parametrize("tiles_k,s", [(256, 8), (10, 3), (2, 2), (3, 8), (1, 1)])
def test_split_k_ranges_partition(tiles_k, s):
    ranges = [oracle.split_k_range(tiles_k, s, p) for p in range(s)]
    pos = 0
    for start, count in ranges:
        assert start == pos and count >= 0
        pos += count
    assert pos == tiles_k
    counts = [c for _, c in ranges]
    assert max(counts) - min(counts) <= 1 and counts == sorted(counts, reverse=True)


def test_swizzle_known_answer_and_bijection():
    # the reference's sm_86 A stage [64, 16] f16: perPhase 4, maxPhase 2,
    # 16-byte span (8 elems), minor extent 16 (test/Transforms/exact_direct_contract.mlir:14)
    for row in range(8):
        phase = (row // 4) % 2
        for col in range(16):
            want = ((col // 8) ^ phase) * 8 + col % 8
            assert oracle.swizzle_minor(row, col, 4, 2, 8, 16) == want
    # gfx950 [*, 64] f16 stage rows: 8 chunks of 8, perPhase 1, maxPhase 8
    for row in range(64):
        perm = [oracle.swizzle_minor(row, c, 1, 8, 8, 64) for c in range(64)]
        assert sorted(perm) == list(range(64))
    assert oracle.swizzle_minor(5, 3, 1, 1, 8, 64) == 3  # maxPhase 1: identity


def _bank_conflict_ways(addrs, bytes_per_lane, lanes_per_cycle):
    """Brute-force LDS bank model of gfx950 (64 banks x 4 bytes): the lanes
    of one cycle are served together; the cycle's cost is the largest number
    of distinct 4-byte words any one bank must deliver."""
    worst = 1
    for c0 in range(0, len(addrs), lanes_per_cycle):
        words = {}
        for a in addrs[c0:c0 + lanes_per_cycle]:
            for w in range(a // 4, (a + bytes_per_lane) // 4):
                words.setdefault(w % 64, set()).add(w)
        worst = max(worst, max(len(v) for v in words.values()))
    return worst


def _mfma16_b_read_addrs(second_term):
    """Byte addresses of one ds_read_b64_tr_b16 of the 16x16x32 B fragment
    (tile jj = 0, k step 0, first half) in a [64][256] f16 stage: lane l reads
    k row 8 (l/16) + (l%16)/4, columns 4 (l%4) .. +3, through the plan's
    swizzle (64-byte segments XOR k % 4; optionally 32-byte units XOR
    (k / 8) % 2)."""
    addrs = []
    for lane in range(64):
        k = 8 * (lane // 16) + (lane % 16) // 4
        n = 4 * (lane % 4)
        if second_term:
            phys = oracle.swizzle_minor2(k, n, 1, 4, 32, 8, 2, 16, 256)
        else:
            phys = oracle.swizzle_minor(k, n, 1, 4, 32, 256)
        addrs.append(k * 512 + phys * 2)
    return addrs


def test_second_swizzle_term_bijection_and_bank_conflicts():
    """The gfx950 second XOR term keeps every row a permutation, reduces to
    the reference's swizzle when off, and makes the 16x16x32 B read
    conflict-free: without it the two 16-lane groups of a cycle (k rows 8
    apart, same k % 4) hit the same banks, a 2-way conflict (what the
    SQ_LDS_BANK_CONFLICT counter showed on the GPU)."""
    for k in range(64):
        perm = [oracle.swizzle_minor2(k, n, 1, 4, 32, 8, 2, 16, 256) for n in range(256)]
        assert sorted(perm) == list(range(256))
        # the second term moves whole 16-column (32-byte) units inside a
        # 32-column (64-byte) segment of the first
        for n in range(0, 256, 16):
            assert perm[n] // 32 == oracle.swizzle_minor(k, n, 1, 4, 32, 256) // 32
        assert [oracle.swizzle_minor2(k, n, 1, 4, 32, 8, 1, 16, 256) for n in range(256)] == \
            [oracle.swizzle_minor(k, n, 1, 4, 32, 256) for n in range(256)]
    # closed form of the encoding: chunk' = chunk ^ 4 (k % 4) ^ 2 ((k / 8) % 2)
    for k in range(32):
        for chunk in range(32):
            got = oracle.swizzle_minor2(k, 8 * chunk, 1, 4, 32, 8, 2, 16, 256) // 8
            assert got == chunk ^ (4 * (k % 4)) ^ (2 * ((k // 8) % 2))
    assert _bank_conflict_ways(_mfma16_b_read_addrs(False), 8, 32) == 2
    assert _bank_conflict_ways(_mfma16_b_read_addrs(True), 8, 32) == 1


def _f32_epilogue_lds(swizzle=True):
    """Byte addresses of the 16x16x32 instance's f32 C epilogue in one wave's
    8 KiB LDS block (one 16-row block of the wave's 128x128 tile, 512-byte
    rows): the ds_write_b128 of tile j by lane l (row l % 16, columns
    16 j + 4 (l / 16) .. +3, chunk c = 4 j + l / 16 at c ^ row) and the
    ds_read_b128 t by lane l (row 2 t + l / 32, chunk l % 32 at chunk ^ row)."""
    sw = (lambda c, r: c ^ r) if swizzle else (lambda c, r: c)
    writes = {j: [(l % 16) * 512 + sw(4 * j + l // 16, l % 16) * 16 for l in range(64)]
              for j in range(8)}
    reads = {t: [(2 * t + l // 32) * 512 + sw(l % 32, 2 * t + l // 32) * 16
                 for l in range(64)] for t in range(8)}
    return writes, reads


def test_f32_epilogue_lds_map():
    """The f32 C epilogue of the 16x16x32 instance: every element is written
    to its own 16 bytes of the block, each whole-row read returns the row and
    columns it stores, and both directions are free of bank conflicts at 16
    lanes of 16 bytes per cycle. The chunk ^ row term is what makes them so:
    without it a quarter wave's 16 rows share one bank group, 16-way."""
    writes, reads = _f32_epilogue_lds()
    held = {}
    for j, addrs in writes.items():
        for l, a in enumerate(addrs):
            assert a % 16 == 0 and 0 <= a < 8192
            held[a] = (l % 16, 16 * j + 4 * (l // 16))  # (row, first column)
    assert len(held) == 8 * 64  # a bijection onto the 512 chunks of the block
    for t, addrs in reads.items():
        for l, a in enumerate(addrs):
            assert held[a] == (2 * t + l // 32, 4 * (l % 32))
    for addrs in list(writes.values()) + list(reads.values()):
        assert _bank_conflict_ways(addrs, 16, 16) == 1
    plain_w, plain_r = _f32_epilogue_lds(swizzle=False)
    assert _bank_conflict_ways(plain_w[0], 16, 16) == 16
    assert _bank_conflict_ways(plain_r[0], 16, 16) == 1  # reads are whole rows either way
