"""The oracle pinned against what it did not write (CPU).

Each check names what pins it: the vllm-exl3 golden (tests/golden/exl3_golden.npz, a byte copy of the reference's
common/tests/data/exl3_golden.npz), the reference's hand-computed values (common/tests/exl3_decode_test.c:51-106),
the reference's own C compiled from /root/reference into oracle/_ref (this container only), closed forms of the
mathematics, and brute force. Every comparison has a negative control that shows it can fail.
"""
import ctypes as C
import os

import numpy as np
import pytest

import oracle

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "exl3_golden.npz")


def _golden():
    z = np.load(GOLDEN, allow_pickle=False)
    for bits in (3, 4):
        for cb in ("mcg", "mul1"):
            yield bits, cb, z[f"trellis_k{bits}_{cb}"], z[f"w_hat_k{bits}_{cb}"].view(np.uint16)


# ------------------------------------------------------------------------------------------ golden (vllm-exl3)
def test_trellis_decode_is_bit_exact_against_the_vllm_exl3_golden(oracle_lib):
    n = 0
    for bits, cb, tr, wh in _golden():
        got = oracle.trellis_decode(tr, bits, cb)
        assert got.shape == wh.shape
        assert np.array_equal(got, wh), f"K={bits} {cb}"
        n += 1
    assert n == 4


def test_the_golden_comparison_can_fail(oracle_lib):
    bits, cb, tr, wh = list(_golden())[3]          # K=4 mul1
    t = tr.copy().view(np.uint16)
    t.reshape(-1)[5] ^= 0x0100
    assert not np.array_equal(oracle.trellis_decode(t, bits, cb), wh)
    assert not np.array_equal(oracle.trellis_decode(tr, bits, "mcg"), wh)
    assert not np.array_equal(oracle.trellis_decode(tr, bits, "3inst"), wh)


# ------------------------------------------------------------------------------------------ hand values
HAND = [(0x0000, 0x3A25, 0x3F60, 0xC2E8), (0x0001, 0xBB5B, 0x304E, 0x3921),
        (0x1234, 0xC066, 0x3E0F, 0xB89E), (0xFFFF, 0xB110, 0x3ACD, 0xB936)]


def test_codebooks_give_the_hand_computed_values(oracle_lib):
    for st, i3, mcg, mul1 in HAND:
        assert oracle.codebook_value(st, "3inst") == i3
        assert oracle.codebook_value(st, "mcg") == mcg
        assert oracle.codebook_value(st, "mul1") == mul1
    assert oracle.codebook_value(0x10000, "mul1") == 0xC2E8
    assert oracle.codebook_value(0, 7) == 0x7E00


def test_mul1_closed_form_over_all_states(oracle_lib):
    """mul1 from its definition in float64 numpy, independently: fp16((1024 + bytesum(x * 0x83DCD12D)) * K_INV + K_BIAS)
    with one rounding (numpy's float64 -> float16 cast is round-to-nearest-even)."""
    x = np.arange(65536, dtype=np.uint64)
    h = (x * 0x83DCD12D) & 0xFFFFFFFF
    s = (h & 255) + ((h >> 8) & 255) + ((h >> 16) & 255) + (h >> 24)
    kinv = float(np.uint16(0x1EEE).view(np.float16))
    kbias = float(np.uint16(0xC931).view(np.float16))
    want = ((1024.0 + s.astype(np.float64)) * kinv + kbias).astype(np.float16).view(np.uint16)
    got = oracle.codebook_table("mul1")
    assert np.array_equal(got, want)
    assert not np.array_equal(got, oracle.codebook_table("mcg"))


def test_lop_codebooks_closed_form_over_all_states(oracle_lib):
    x = np.arange(65536, dtype=np.uint64)
    for cb, h in (("mcg", (x * 0xCBAC1FED) & 0xFFFFFFFF), ("3inst", (x * 89226354 + 64248484) & 0xFFFFFFFF)):
        h = (h & 0x8FFF8FFF) ^ 0x3B603B60
        lo = (h & 0xFFFF).astype(np.uint16).view(np.float16).astype(np.float64)
        hi = (h >> 16).astype(np.uint16).view(np.float16).astype(np.float64)
        want = (lo + hi).astype(np.float16).view(np.uint16)
        assert np.array_equal(oracle.codebook_table(cb), want), cb


def test_a_hand_built_3inst_tile_decodes_by_the_formula(oracle_lib):
    sym = np.arange(256, dtype=np.uint8)
    tile = oracle.tile_pack(sym, 8)
    st = oracle.tile_states(sym, 8)
    assert st[0] == 0xFF00 and st[1] == 0x0001 and st[0x35] == 0x3435
    w = oracle.trellis_decode(tile.reshape(1, 1, -1), 8, "3inst")
    r, c = oracle.pos_to_tile(1)
    assert w[r, c] == 0xBB5B
    for p in range(256):
        r, c = oracle.pos_to_tile(p)
        assert w[r, c] == oracle.codebook_value(int(st[p]), "3inst")


def test_the_tile_map_is_the_stated_one_and_a_bijection(oracle_lib):
    assert oracle.pos_to_tile(0) == (0, 0)
    assert oracle.pos_to_tile(2) == (8, 0)
    assert oracle.pos_to_tile(3) == (9, 0)
    assert oracle.pos_to_tile(4) == (0, 8)
    assert oracle.pos_to_tile(8) == (2, 0)
    assert oracle.pos_to_tile(32) == (0, 1)
    assert oracle.pos_to_tile(255) == (15, 15)
    seen = set()
    for p in range(256):
        r, c = oracle.pos_to_tile(p)
        assert oracle.tile_to_pos(r, c) == p
        seen.add((r, c))
    assert len(seen) == 256


def test_the_tile_stream_is_msb_first_little_endian_words(oracle_lib):
    sym = np.zeros(256, np.uint8)
    sym[0] = 0x9
    t = oracle.tile_pack(sym, 4)
    assert t[1] == 0x9000 and t[0] == 0
    rng = np.random.default_rng(1)
    for bits in range(1, 9):
        s = rng.integers(0, 1 << bits, 256).astype(np.uint8)
        assert np.array_equal(oracle.tile_symbols(oracle.tile_pack(s, bits), bits), s)


def test_states_are_the_window_ending_at_each_symbol(oracle_lib):
    p = np.arange(256)
    sym = ((p * 7 + 3) & 0xF).astype(np.uint8)
    st = oracle.tile_states(sym, 4)
    assert st[10] == (int(sym[7]) << 12 | int(sym[8]) << 8 | int(sym[9]) << 4 | int(sym[10]))
    assert st[1] == (int(sym[254]) << 12 | int(sym[255]) << 8 | int(sym[0]) << 4 | int(sym[1]))
    sym = ((p * 5 + 1) & 0x7).astype(np.uint8)
    st = oracle.tile_states(sym, 3)
    want = (int(sym[15]) << 15 | int(sym[16]) << 12 | int(sym[17]) << 9 | int(sym[18]) << 6 | int(sym[19]) << 3
            | int(sym[20])) & 0xFFFF
    assert st[20] == want


def test_fp16_round_trips_every_finite_half_and_rounds_ties_to_even(oracle_lib):
    L = oracle.lib()
    for h in range(0, 0x10000, 1):
        if (h & 0x7C00) == 0x7C00 and (h & 0x3FF):
            continue
        assert L.or_half_from_double(L.or_half_to_float(h)) == h
    f = oracle.half_from_double
    assert f(1.0 + 2 ** -11) == 0x3C00
    assert f(1.0 + 3 * 2 ** -11) == 0x3C02
    assert f(65504.0) == 0x7BFF and f(65519.0) == 0x7BFF and f(65520.0) == 0x7C00
    assert f(-2 ** -25) == 0x8000
    assert f(2 ** -24 * 1.5) == 0x0002
    # numpy's own float64 -> float16 (RNE) agrees on random doubles across the range
    rng = np.random.default_rng(2)
    xs = rng.standard_normal(2000) * np.exp2(rng.integers(-26, 17, 2000))
    assert all(f(x) == int(np.float16(x).view(np.uint16)) for x in xs)


def _bf16_nearest(bits):
    """bf16 round-to-nearest-even by distance (not by the bit trick): the two bf16 neighbours of each finite f32 as
    float64, the nearer one, ties to the even mantissa; a value past the largest finite bf16's rounding boundary
    becomes inf (IEEE)."""
    b = np.asarray(bits, np.uint32)
    x = b.view(np.float32).astype(np.float64)
    lo = (b >> 16).astype(np.uint32)
    sign = lo & 0x8000
    mag = lo & 0x7FFF
    down = ((sign | mag) << 16).view(np.float32).astype(np.float64)
    up_bits = (sign | (mag + 1)) & 0xFFFF
    up = (up_bits.astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    up = np.where((up_bits & 0x7FFF) == 0x7F80, np.where(sign != 0, -2.0 ** 128, 2.0 ** 128), up)   # inf's place
    dd, du = np.abs(x - down), np.abs(up - x)
    pick_up = (du < dd) | ((du == dd) & ((mag & 1) == 1))
    return np.where(pick_up, up_bits, sign | mag).astype(np.uint16)


def test_bf16_narrowing_is_round_to_nearest_even_with_quiet_nans(oracle_lib):
    """or_f32_to_bf16 (radiance's rad_f32_to_bf16) against the nearest bf16 by distance, over every upper half-word
    with the low halves 0, 1, 0x7FFF, 0x8000, 0x8001, 0xFFFF and random patterns; nans stay nans, quiet, with their
    upper payload; or_f32_to_f16 against numpy's float32 -> float16 (IEEE round to nearest even)."""
    hi = np.arange(1 << 16, dtype=np.uint32) << 16
    lows = np.array([0, 1, 0x7FFF, 0x8000, 0x8001, 0xFFFF], np.uint32)
    rng = np.random.default_rng(11)
    bits = np.concatenate([(hi[:, None] | lows[None, :]).ravel(),
                           rng.integers(0, 1 << 32, size=200000, dtype=np.uint64).astype(np.uint32)])
    bf, h = oracle.narrow(bits.view(np.float32))
    nan = (bits & 0x7FFFFFFF) > 0x7F800000
    fin = (bits & 0x7F800000) != 0x7F800000
    assert np.array_equal(bf[fin], _bf16_nearest(bits[fin]))
    assert np.array_equal(bf[nan], ((bits[nan] >> 16) | 0x40).astype(np.uint16))
    inf = ~nan & ~fin
    assert np.array_equal(bf[inf], (bits[inf] >> 16).astype(np.uint16))
    with np.errstate(over="ignore"):
        want_h = bits[~nan].view(np.float32).astype(np.float16).view(np.uint16)
    assert np.array_equal(h[~nan], want_h)
    # spot values: a tie rounds to even (down, then up), past the largest finite goes to inf
    t = lambda u: int(oracle.narrow(np.array([u], np.uint32).view(np.float32))[0][0])  # noqa: E731
    assert t(0x3F808000) == 0x3F80 and t(0x3F818000) == 0x3F82 and t(0x7F7F8000) == 0x7F80
    # negative control: truncation is not the rule
    assert not np.array_equal(bf[fin], (bits[fin] >> 16).astype(np.uint16))


def test_had128_is_the_normalised_sylvester_hadamard(oracle_lib):
    v = np.zeros(256, np.float32)
    v[0] = 1
    v[129] = 1
    w = oracle.had128(v)
    s = 0.0883883476
    assert np.allclose(w[:128], s, atol=1e-7)
    assert np.allclose(w[128:], np.where(np.arange(128) % 2, -s, s), atol=1e-7)
    rng = np.random.default_rng(3)
    x = (rng.integers(-1000, 1001, 256) / 1000).astype(np.float32)
    assert np.max(np.abs(oracle.had128(oracle.had128(x)) - x)) < 1e-5
    # against scipy's Sylvester Hadamard (natural order) in float64
    from scipy.linalg import hadamard
    H = hadamard(128) / np.sqrt(128)
    y = rng.standard_normal(128).astype(np.float32)
    assert np.max(np.abs(oracle.had128(y) - H @ y.astype(np.float64))) < 1e-5
    with pytest.raises(ValueError):
        oracle.had128(np.zeros(100, np.float32))


def test_codes_plane_elements_are_lsb_first_along_the_row(oracle_lib):
    L = oracle.lib()
    row = np.zeros(8, np.uint8)
    L.or_codes_set(row.ctypes.data, 8, 3, 0, 0, 0x5)
    L.or_codes_set(row.ctypes.data, 8, 3, 0, 2, 0x7)
    assert row[0] == 0xC5 and row[1] == 0x01
    assert L.or_codes_get(row.ctypes.data, 8, 3, 0, 2) == 7
    assert L.or_codes_get(row.ctypes.data, 8, 3, 0, 1) == 0
    assert oracle.row_bytes(2560, 3) == 960 and oracle.row_bytes(640, 4) == 320


@pytest.mark.parametrize("bits", range(1, 9))
def test_w_hat_from_the_plane_equals_w_hat_from_the_trellis(oracle_lib, bits):
    N, K = 64, 48
    rng = np.random.default_rng(10 + bits)
    for cb in ("3inst", "mcg", "mul1"):
        tr = rng.integers(0, 65536, (K // 16) * (N // 16) * 16 * bits).astype(np.uint16)
        wh = oracle.trellis_decode(tr.reshape(K // 16, N // 16, 16 * bits), bits, cb)      # [k][n]
        codes = oracle.record_to_codes(tr, N, K, bits)
        got = oracle.what_rows(codes, N, K, bits, cb, f16=True)                             # [n][k]
        assert np.array_equal(got, wh.T)
        assert np.array_equal(oracle.what_rows(codes, N, K, bits, cb, row0=20, n=9, f16=True), wh.T[20:29])
        assert np.array_equal(oracle.codes_to_record(codes, N, K, bits), tr)


def test_all_zero_codes_give_the_closed_form(oracle_lib):
    """Every state 0 -> W_hat == mul1(0) = 0xC2E8 everywhere; Hb J Hb is 128 c at each 128-block origin and 0 elsewhere,
    so W[n][k] = 128 * (-3.453125) * suh[k] * svh[n] there and ~0 elsewhere (a textbook known answer)."""
    N, K, bits = 256, 256, 4
    codes = np.zeros((N, oracle.row_bytes(K, bits)), np.uint8)
    assert np.all(oracle.what_rows(codes, N, K, bits, "mul1", f16=True) == 0xC2E8)
    rng = np.random.default_rng(4)
    suh = (rng.integers(0, 2, K) * 2 - 1).astype(np.float16)
    svh = (rng.integers(0, 2, N) * 2 - 1).astype(np.float16)
    W = oracle.decode_rows(codes, N, K, bits, "mul1", suh, svh)
    want = np.zeros((N, K))
    for n0 in range(0, N, 128):
        for k0 in range(0, K, 128):
            want[n0, k0] = 128 * -3.453125 * float(suh[k0]) * float(svh[n0])
    assert np.max(np.abs(W - want)) < 1e-3
    assert abs(W[0, 0]) > 400


def test_decode_rows_against_a_float64_dense_product(oracle_lib):
    """W = diag(suh) Hb W_hat Hb diag(svh) in exllamav3's [k, n] terms; here [n][k] = svh[n] (Hb W_hat^T Hb)[n][k]
    suh[k], computed in float64 with scipy's Hadamard; the stacked suh1 rule for the second half of the rows."""
    from scipy.linalg import hadamard
    N, K, bits = 256, 128, 3
    rng = np.random.default_rng(5)
    codes = rng.integers(0, 256, (N, oracle.row_bytes(K, bits))).astype(np.uint8)
    suh = (rng.standard_normal(K) * 0.1).astype(np.float16)
    suh1 = (rng.standard_normal(K) * 0.1).astype(np.float16)
    svh = rng.standard_normal(N).astype(np.float16)
    wh = oracle.what_rows(codes, N, K, bits, "mcg").astype(np.float64)      # [n][k]
    H = hadamard(128) / np.sqrt(128)
    Hn = np.kron(np.eye(N // 128), H)
    Hk = np.kron(np.eye(K // 128), H)
    s = np.where(np.arange(N)[:, None] >= N // 2, suh1.astype(np.float64)[None, :], suh.astype(np.float64)[None, :])
    want = (Hn @ ((wh @ Hk) * s)) * svh.astype(np.float64)[:, None]
    got = oracle.decode_rows(codes, N, K, bits, "mcg", suh, svh, suh1=suh1)
    assert np.max(np.abs(got - want)) <= 1e-5 * np.max(np.abs(want))
    bad = oracle.decode_rows(codes, N, K, bits, "mcg", suh1, svh, suh1=suh)   # swapped halves: a control
    assert np.max(np.abs(bad - want)) > 1e-2 * np.max(np.abs(want))


def test_moe_scatter_is_a_stable_counting_sort(oracle_lib):
    import exl3c4_synth as syn
    rng = np.random.default_rng(6)
    for n_tok, top_k, E, base in ((8, 10, 512, 0), (37, 4, 16, 3), (5, 2, 4, 0)):
        ids = rng.integers(-2, E + base + 2, (n_tok, top_k)).astype(np.int32)
        st, off = oracle.moe_scatter(ids, E, base)
        flat = ids.reshape(-1) - base
        keep = np.nonzero((flat >= 0) & (flat < E))[0]
        want = keep[np.argsort(flat[keep], kind="stable")]
        assert np.array_equal(st[: want.size], want) and np.all(st[want.size:] == -1)
        assert off[0] == 0 and off[-1] == want.size
        assert np.array_equal(np.diff(off), np.bincount(flat[keep], minlength=E))
        st2, off2 = syn.moe_scatter(ids, E, base)
        assert np.array_equal(st, st2) and np.array_equal(off, off2)


# ------------------------------------------------------------------------------------------ against the reference C
class _View(C.Structure):
    _fields_ = [("rows", C.c_int64), ("cols", C.c_int64), ("bits", C.c_int), ("codebook", C.c_int),
                ("codes", C.c_void_p), ("codes_row_bytes", C.c_int64), ("suh", C.c_void_p), ("suh1", C.c_void_p),
                ("svh", C.c_void_p)]


def test_codebooks_equal_the_reference_c_on_every_state(oracle_lib, ref_common):
    ref_common.exl3_codebook_value.restype = C.c_uint16
    ref_common.exl3_codebook_value.argtypes = [C.c_uint32, C.c_int]
    for cb in range(3):
        ours = oracle.codebook_table(cb)
        theirs = np.array([ref_common.exl3_codebook_value(s, cb) for s in range(65536)], np.uint16)
        assert np.array_equal(ours, theirs), cb


@pytest.mark.parametrize("bits", range(1, 9))
def test_trellis_decode_and_layout_equal_the_reference_c(oracle_lib, ref_common, bits):
    rng = np.random.default_rng(100 + bits)
    kt, nt = 3, 4
    L = ref_common
    L.exl3_trellis_decode.restype = C.c_int
    L.exl3_trellis_decode.argtypes = [C.c_void_p, C.c_int64, C.c_int64, C.c_int, C.c_int, C.c_void_p]
    L.exl3_record_to_codes.argtypes = [C.c_void_p, C.c_int64, C.c_int64, C.c_int, C.c_void_p, C.c_int64]
    for cb in range(3):
        tr = rng.integers(0, 65536, kt * nt * 16 * bits).astype(np.uint16)
        ref = np.zeros((16 * kt, 16 * nt), np.uint16)
        assert L.exl3_trellis_decode(tr.ctypes.data, kt, nt, bits, cb, ref.ctypes.data) == 0
        assert np.array_equal(oracle.trellis_decode(tr.reshape(kt, nt, -1), bits, cb), ref)
        rows, cols = 16 * nt, 16 * kt
        rb = oracle.row_bytes(cols, bits)
        rc = np.zeros((rows, rb), np.uint8)
        L.exl3_record_to_codes(tr.ctypes.data, rows, cols, bits, rc.ctypes.data, rb)
        assert np.array_equal(oracle.record_to_codes(tr, rows, cols, bits), rc)


def test_had128_and_decode_rows_equal_the_reference_c_to_the_bit(oracle_lib, ref_common):
    L = ref_common
    L.exl3_had128.argtypes = [C.c_void_p, C.c_int64]
    L.exl3_decode_rows.argtypes = [C.POINTER(_View), C.c_int64, C.c_int64, C.c_void_p]
    rng = np.random.default_rng(7)
    v = rng.standard_normal(512).astype(np.float32)
    r = v.copy()
    L.exl3_had128(r.ctypes.data, 512)
    assert np.array_equal(oracle.had128(v).view(np.uint32), r.view(np.uint32))
    N, K, bits = 256, 256, 4
    codes = rng.integers(0, 256, (N, oracle.row_bytes(K, bits))).astype(np.uint8)
    suh = (rng.standard_normal(K) * 0.1).astype(np.float16)
    suh1 = (rng.standard_normal(K) * 0.1).astype(np.float16)
    svh = rng.standard_normal(N).astype(np.float16)
    out = np.zeros((N, K), np.float32)
    vw = _View(N, K, bits, 2, codes.ctypes.data, 0, suh.ctypes.data, suh1.ctypes.data, svh.ctypes.data)
    assert L.exl3_decode_rows(C.byref(vw), 0, N, out.ctypes.data) == 0
    got = oracle.decode_rows(codes, N, K, bits, "mul1", suh, svh, suh1=suh1)
    assert np.array_equal(got.view(np.uint32), out.view(np.uint32))
