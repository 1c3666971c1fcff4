"""The drop-in boundary's host-side contract (CPU: nothing is launched).

- Every kernel in libexl3c4.so fits the radiance engine's 768-byte kernel-argument slot, hidden arguments included,
  and no kernel taking the op argument block reads a hidden argument (kernels/exl3r4d/exl3r4d_dev.h:5-6,
  tests/gpu/kernarg_check.sh: the engine refuses a larger segment at dispatch, which hipLaunchKernel never shows).
- Scratch sized once from the parameters at the band top (docs/STEP0.md:142-146) takes every smaller batch.
- The size queries answer for every op a launch accepts; the tables' strides are refused like the launch refuses them.
"""
import ctypes as C
import os

import pytest

import exl3c4
import kernarg
from hostops import Fake, op

LIB = os.path.join(os.path.dirname(exl3c4.__file__), "libexl3c4.so")


# ------------------------------------------------------------------------------------------ kernel arguments
@pytest.fixture(scope="module")
def kernels():
    if not kernarg.tools_present():
        pytest.skip("objcopy / llvm-readelf absent")
    ks = kernarg.kernels(LIB)
    assert ks, "no kernel metadata found in the library's code objects"
    return ks


def test_every_kernel_fits_the_engine_kernel_argument_slot(kernels):
    big = [(k["name"], k["kernarg"]) for k in kernels if k["kernarg"] > 768]
    assert not big, f"argument segments over 768 bytes: {big[:5]}"


def test_the_op_kernels_take_the_compact_block_and_no_hidden_argument(kernels):
    ops = [k for k in kernels if "Exl3c4Launch" in k["name"]]
    names = {k["name"].split("ILi")[0].split("E12Exl3c4Launch")[0][-8:] for k in ops}
    # every op kernel: prep, gate_up's and down's GEMMs, the epilogue, gate_up_down's single kernel, the prefill ones
    for want in ("k_prep", "k_gepi", "k_gu", "k_dn", "k_gd", "k_plan", "k_rot", "k_gu_pf", "k_dn_pf"):
        assert any(n.endswith(want) for n in names), want
    assert len(ops) >= 7 * 3 * 5                       # 7 K x 3 codebooks for each templated GEMM kernel
    for k in ops:
        assert k["by_value"] == [632], (k["name"], k["by_value"])
        assert not k["hidden"], f"{k['name']} reads hidden arguments {k['hidden']}"
        assert k["kernarg"] == 632


def test_the_hidden_argument_reading_is_seen_where_it_happens(kernels):
    """Negative control of the check above: the routing kernels read blockDim / gridDim, and the metadata shows it."""
    route = [k for k in kernels if "k_scatter" in k["name"] or "k_route_scatter" in k["name"]]
    assert route and all(k["hidden"] for k in route)
    assert all(k["kernarg"] > sum(k["by_value"]) for k in route)


# ------------------------------------------------------------------------------------------ scratch at the band top
BANDS = [
    # (op, H, W, E, M, top_k): the configs' geometries and the reference's band tops (test_exl3ref.py:1282-1300)
    (exl3c4.GU_DN, 2048, 512, 512, 8, 10),       # configs[2]: the decode layer
    (exl3c4.GU_DN, 2048, 512, 1, 64, 1),         # configs[1]: one expert, a band of 64 tokens
    (exl3c4.GATE_UP, 2048, 512, 512, 16, 10),    # the decode band top M = 16
    (exl3c4.DOWN, 2048, 512, 512, 16, 10),
    (exl3c4.GU_DN, 2560, 640, 512, 16, 10),      # the reference's per-rank geometry
    (exl3c4.GU_DN, 2048, 512, 512, 96, 10),      # a band across the prefill threshold (448 rows here)
]


@pytest.mark.parametrize("which,H,W,E,M,top_k", BANDS)
def test_band_top_scratch_takes_every_smaller_batch(which, H, W, E, M, top_k):
    """exl3c4_scratch_bytes at the band top is at least what a launch of every T' <= M top_k rows needs
    (exl3c4_launch_scratch_bytes, exl3c4_launch's refusal threshold). The split-K count of the decode GEMV grows as T
    shrinks, so this is not a monotone function; a single size at the top must still cover it."""
    band = exl3c4.scratch_bytes(op(which, H=H, W=W, E=E, M=M, top_k=top_k))
    assert band > 0
    geom = exl3c4.lib().exl3c4_scratch_bytes_geom(
        which, 1, (C.c_int32 * 4)(*([2 * W if which != exl3c4.DOWN else H] * 4)),
        (C.c_int32 * 4)(*([H if which != exl3c4.DOWN else W] * 4)), M, top_k, E)
    assert geom == band                          # the plugin's hook gives the same size from the parameters alone
    needs = [exl3c4.launch_scratch_bytes(op(which, H=H, W=W, E=E, M=M, top_k=top_k, rows_T=t))
             for t in range(1, M * top_k + 1)]
    assert min(needs) > 0 and max(needs) <= band
    assert max(needs) == band                    # and no more than the largest of them


def test_the_carve_is_not_monotone_so_the_band_top_alone_would_not_do():
    """Why the maximum is needed (the control): one expert with a band of 64 tokens -- 64 rows take the prefill path,
    63 the decode path, whose partial sums at its split-K need more than three times the band top's carve."""
    n63 = exl3c4.launch_scratch_bytes(op(exl3c4.GU_DN, H=2048, W=512, E=1, M=64, top_k=1, rows_T=63))
    n64 = exl3c4.launch_scratch_bytes(op(exl3c4.GU_DN, H=2048, W=512, E=1, M=64, top_k=1, rows_T=64))
    assert n63 > 3 * n64
    assert exl3c4.scratch_bytes(op(exl3c4.GU_DN, H=2048, W=512, E=1, M=64, top_k=1)) >= n63


@pytest.mark.parametrize("which,a_rot", [(exl3c4.DOWN, 0), (exl3c4.GATE_UP, 1)])
def test_size_queries_answer_for_sorted_row_inputs_below_the_band_top(which, a_rot):
    """down and gate_up(a_rot 1) read T sorted rows: a launch of T < M top_k rows is accepted, and the band's size
    queries answer for it too (they size from the geometry, not from this launch's x)."""
    o = op(which, M=8, top_k=10, E=64, a_rot=a_rot, rows_T=50)
    assert exl3c4.launch_scratch_bytes(o) > 0
    assert exl3c4.scratch_bytes(o) >= exl3c4.launch_scratch_bytes(o)
    assert exl3c4.scratch_bytes(o) == exl3c4.scratch_bytes(op(which, M=8, top_k=10, E=64, a_rot=a_rot))


# ------------------------------------------------------------------------------------------ stride refusals
def _rc(o):
    return exl3c4.lib().exl3c4_launch(C.byref(o), C.c_void_p(0x100000), 1 << 40, None)


def test_down_tables_of_gate_up_down_are_refused_like_gate_up_tables():
    o = op(exl3c4.GU_DN, H=256, W=128, E=4)
    o.dn[0].codes_stride = 256 * 128 * 4 // 8 - 4          # below one [H, W] record at K = 4
    assert _rc(o) == -4
    o = op(exl3c4.GU_DN, H=256, W=128, E=4)
    o.dn[0].svh_stride = 2 * 256 - 2                        # below svh [H]
    assert _rc(o) == -4
    o = op(exl3c4.GATE_UP, H=256, W=128, E=4)
    o.cls[0].codes_stride = 256 * 256 * 4 // 8 - 4          # the same for gate_up's own table
    assert _rc(o) == -4
    o = op(exl3c4.GATE_UP, H=256, W=128, E=4)
    o.cls[0].svh_stride = 2 * 256 - 2
    assert _rc(o) == -4
    o = op(exl3c4.GATE_UP, H=256, W=128, E=4)
    o.cls[0].suh1_stride = 2 * 256 - 2
    assert _rc(o) == -4


def test_pitches_and_strides_past_32_bits_are_refused():
    """The kernels' argument block holds pitches and table strides in 32 bits; the host refuses larger ones."""
    o = op(exl3c4.GATE_UP, E=4)
    o.x_pitch = 1 << 31
    assert _rc(o) == -4
    o = op(exl3c4.GATE_UP, E=4)
    o.y_pitch = 1 << 31
    assert _rc(o) == -4
    o = op(exl3c4.GATE_UP, E=4)
    o.cls[0].codes_stride = 1 << 31
    assert _rc(o) == -4
    o = op(exl3c4.GU_DN, E=4)
    o.dn[0].codes_stride = 1 << 31
    assert _rc(o) == -4


def test_an_accepted_op_reaches_the_scratch_check():
    """The control of the refusals above: the same ops unmodified pass every check and stop only at the scratch."""
    for which in (exl3c4.GATE_UP, exl3c4.GU_DN, exl3c4.DOWN):
        o = op(which, E=4)
        assert exl3c4.lib().exl3c4_launch(C.byref(o), None, 0, None) == -20
    assert Fake((2, 3)).numel() == 6


def test_input_pitches_past_the_prefill_offsets_keep_the_decode_kernels():
    """The prefill GEMMs address a chunk's staged rows by 32-bit byte offsets from a wave-uniform base, so the prefill
    path takes input pitches up to 2^24 halves; past that a launch of any T runs on the decode kernels, and its
    scratch is theirs (the split-K partial sums), not the prefill path's (the plan, the rotated input)."""
    T = 96 * 10
    assert exl3c4.is_prefill(T, 512)

    def sized(pitch):
        o = op(exl3c4.GU_DN, H=2048, W=512, E=512, M=96, top_k=10)
        o.x_pitch = pitch
        return exl3c4.launch_scratch_bytes(o)

    at, past = sized(1 << 24), sized((1 << 24) + 64)
    assert sized(2048) == at                     # within the bound: the prefill path, whatever the pitch
    assert past > 0 and past != at
    small = op(exl3c4.GU_DN, H=2048, W=512, E=512, M=96, top_k=10, rows_T=T)
    assert exl3c4.launch_scratch_bytes(small) == at
