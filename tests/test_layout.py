"""The stored form, the exported symbols and the host refusals of libexl3c4.so (CPU: no kernel is launched)."""
import ctypes as C
import os
import re

import numpy as np
import pytest

import exl3c4
import exl3c4_synth as syn
import oracle

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def expected_record(codes, rows, cols, bits):
    """The stored record built from the ORACLE's exllamav3 record by the documented permutation: block (nb, ks),
    segment X = c + 16 g (c = 2 s + t) = words [s K, s K + K) of tile (4 ks + g, 2 nb + t)."""
    rec = oracle.codes_to_record(codes, rows, cols, bits)                 # u16 [kt][nt][16K]
    kt, nt = cols // 16, rows // 16
    words = rec.view(np.uint32).reshape(kt, nt, 8, bits)                  # [tk][tn][s][K]
    nbs, kss = rows // 32, cols // 64
    X = np.arange(64)
    c, g = X % 16, X // 16
    s, t = c // 2, c % 2
    out = np.empty((nbs, kss, 64, bits), np.uint32)
    for nb in range(nbs):
        for ks in range(kss):
            out[nb, ks] = words[4 * ks + g, 2 * nb + t, s]
    return out.reshape(-1).view(np.uint8)


@pytest.mark.parametrize("bits", range(1, 9))
def test_relayout_is_the_documented_permutation_of_the_oracle_record(bits):
    rng = np.random.default_rng(bits)
    rows, cols = 64, 128
    codes = syn.random_codes(rng, rows, cols, bits)
    got = exl3c4.relayout(codes, rows, cols, bits)
    assert np.array_equal(got, expected_record(codes, rows, cols, bits))
    assert np.array_equal(exl3c4.unrelayout(got, rows, cols, bits), codes)


def test_relayout_round_trip_at_the_expert_geometry():
    rng = np.random.default_rng(11)
    for rows, cols, bits in ((1024, 2048, 4), (2048, 512, 3), (256, 128, 8), (512, 256, 2)):
        codes = syn.random_codes(rng, rows, cols, bits)
        rec = exl3c4.relayout(codes, rows, cols, bits)
        assert rec.size == exl3c4.lib().exl3c4_record_bytes(rows, cols, bits)
        assert np.array_equal(exl3c4.unrelayout(rec, rows, cols, bits), codes)
        flipped = rec.copy()
        flipped[rec.size // 2] ^= 0x10                                     # a control: one bit moves the plane
        assert not np.array_equal(exl3c4.unrelayout(flipped, rows, cols, bits), codes)


def test_relayout_refuses_what_it_cannot_hold():
    codes = np.zeros((64, 64), np.uint8)
    with pytest.raises(ValueError):
        exl3c4.relayout(codes, 48, 128, 4)     # rows % 32
    with pytest.raises(ValueError):
        exl3c4.relayout(codes, 64, 96, 4)      # cols % 64
    with pytest.raises(ValueError):
        exl3c4.relayout(codes, 64, 128, 9)     # K


def test_the_library_exports_every_declared_entry_point():
    text = open(os.path.join(ROOT, "include", "exl3c4.h")).read()
    declared = set(re.findall(r"\b(exl3c4_[a-z0-9_]+)\s*\(", text))
    assert len(declared) >= 8
    L = exl3c4.lib()
    for name in sorted(declared):
        assert hasattr(L, name), name
    assert L.exl3c4_build_target() == b"gfx950"
    assert L.exl3c4_abi_version() == 1


# ------------------------------------------------------------------------------------------ refusals (host only)
from hostops import Fake as _T, op as _op  # noqa: E402


def _launch_rc(o, scratch=None, nbytes=0):
    return exl3c4.lib().exl3c4_launch(C.byref(o), scratch, nbytes, None)


def test_refusals_are_decided_on_the_host_before_any_write():
    assert _launch_rc(_op(bits=9)) == -2                      # RAD_E_DTYPE: K outside 2..8
    assert _launch_rc(_op(bits=1)) == -2
    assert _launch_rc(_op(cb=7)) == -2                        # unknown codebook
    assert _launch_rc(_op(h_rot=2)) == -12                    # RAD_E_INVAL
    assert _launch_rc(_op(a_rot=3)) == -12
    assert _launch_rc(_op(H=200)) == -1                       # RAD_E_SHAPE: K % 128
    assert _launch_rc(_op(W=64)) == -1                        # gate_up N % 256
    assert _launch_rc(_op(ycols=64)) == -1                    # output not exactly the op's width
    assert _launch_rc(_op(op=exl3c4.DOWN, ycols=128)) == -1
    assert _launch_rc(_op(xcols=128)) == -1                   # input narrower than K
    assert _launch_rc(_op(M=0)) == -1
    assert _launch_rc(_op()) == -20                           # RAD_E_SCRATCH: none given
    o = _op(op=exl3c4.DOWN)
    o.cls[0].codes = None
    assert _launch_rc(o) == -12                               # a required table absent
    o = _op(h_rot=1)
    o.cls[0].dn_suh = None
    assert _launch_rc(o) == -12                               # gate_up h_rot = 1 needs dn_suh
    o = _op(op=exl3c4.GU_DN)
    o.dn[0].rows = 128
    assert _launch_rc(o) == -1                                # gate_up_down's down geometry is [K, N / 2]


def test_down_k_apart_is_checked_on_the_host():
    """Exl3c4Op.dn_bits (gate_up_down's down K, 0 = bits): K outside 2..8 refused, another op given one refused, and
    down's record stride held against down's own K."""
    o = _op(op=exl3c4.GU_DN)
    o.dn_bits = 9
    assert _launch_rc(o) == -2                                # RAD_E_DTYPE
    o.dn_bits = 1
    assert _launch_rc(o) == -2
    o = _op(op=exl3c4.GATE_UP)
    o.dn_bits = 3
    assert _launch_rc(o) == -12                               # RAD_E_INVAL: only gate_up_down has a down K
    o = _op(op=exl3c4.GU_DN)
    o.dn_bits = o.bits
    assert _launch_rc(o) == -20                               # the same K spelt out: accepted up to the scratch
    o = _op(op=exl3c4.GU_DN, bits=2)
    o.dn_bits = 8
    rb = exl3c4.lib().exl3c4_record_bytes
    rb.restype, rb.argtypes = C.c_int64, [C.c_int64, C.c_int64, C.c_int32]
    o.dn[0].codes_stride = rb(o.dn[0].rows, o.dn[0].cols, 2)
    assert _launch_rc(o) == -4                                # RAD_E_STRIDE: a K = 2 entry cannot hold K = 8
    o.dn[0].codes_stride = rb(o.dn[0].rows, o.dn[0].cols, 8)
    assert _launch_rc(o) == -20


def test_scratch_is_sized_from_the_parameters_alone():
    o = _op(M=8, top_k=10, E=64)
    n1 = exl3c4.scratch_bytes(o)
    o.T = 5                                                   # the actual row count does not shrink it
    assert exl3c4.scratch_bytes(o) == n1 and n1 > 0
    assert exl3c4.scratch_bytes(_op(M=16, top_k=10, E=64)) > n1
    assert exl3c4.scratch_bytes(_op(bits=9)) == -2


def test_launch_gather_refuses_like_launch_and_moe_gather():
    L = exl3c4.lib()
    w, r, out = C.c_void_p(0x20000), C.c_void_p(0x30000), C.c_void_p(0x40000)

    def rc(o, out_=out, pitch=256, w_=w):
        return L.exl3c4_launch_gather(C.byref(o), None, 0, None, None, 0, w_, r, out_, pitch)
    assert rc(_op(op=exl3c4.GU_DN, bits=9)) == -2             # the op's own refusals first
    assert rc(_op(op=exl3c4.GATE_UP)) == -12                  # y must be down's output
    assert rc(_op(op=exl3c4.GU_DN), w_=None) == -12
    assert rc(_op(op=exl3c4.GU_DN), pitch=128) == -4          # moe_gather's: out narrower than y
    assert rc(_op(op=exl3c4.GU_DN), out_=C.c_void_p(0x40008)) == -3
    assert rc(_op(op=exl3c4.GU_DN), w_=C.c_void_p(0x20002)) == -3
    assert rc(_op(op=exl3c4.GU_DN)) == -20                    # then the scratch
    o = _op(op=exl3c4.GU_DN, M=8, top_k=10, E=64)
    assert exl3c4.ctr_bytes(o) >= (80 + 1 + 8) * 256          # a counter line a row and a token

