"""Down's epilogue and the kernels' narrowing conversions, held to the bit (GPU).

The reference holds down's output to the bit (tests/ref/test_exl3ref.py:336-346) with a stated round-to-nearest-even
bf16 (kernels/exl3r4d/exl3r4d_common.hip.h:164-167). The device's f32 accumulations may differ from the oracle's
ascending sums (the MFMA adds in another order), so the epilogue is isolated: the oracle's down epilogue -- had128 of
each 128-column block, x svh, round to bf16 (kernels/exl3ref/ref.c:213-225; oracle or_had128, or_f32_to_bf16) --
applied to the DEVICE's own f32 accumulations must give the device's y bit for bit, on every path that forms y:
  the decode pair's down (k_dn), gate_up_down's single kernel (k_gd), and the prefill GEMM (k_dn_pf, read through
  exl3c4_launch_checked, which also leaves its sums).
The conversions themselves (down's one v_cvt_pk_bf16_f32 for two values, h's f32 -> f16) run through the checker
entry exl3c4_check_narrow over every upper half-word of an f32 with the low halves 0, 1, 0x7FFF, 0x8000, 0x8001 and
0xFFFF (each nan class, the ties, the denormals, the overflow to inf) against the oracle's rules.
"""
import numpy as np
import pytest

import oracle
from cases import Case, Dev, narrowed_ok
from gpuchecks import say

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def torch_cuda():
    torch = pytest.importorskip("torch")
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import exl3c4
    exl3c4.lib()          # raises if the library is not built: no fallback exists
    return torch


def oracle_down_epilogue(case, dacc):
    """y bf16 bits [T, N] from down's f32 accumulations [T, >= N] through the oracle's epilogue: every live row's
    had128 per 128-block, x svh (f32), or_f32_to_bf16; rows no run holds and negative sorted_tok zero; a narrower
    class's tail zero."""
    N = max(d.rows for d in case.dn)
    y = np.zeros((case.T, N), np.uint16)
    for e, rows in case.live_rows().items():
        d = case.dn[e]
        sv = np.asarray(d.svh).view(np.float16).astype(np.float32)
        v = oracle.had128(np.ascontiguousarray(dacc[rows, :d.rows], np.float32).ravel()).reshape(len(rows), d.rows)
        bf, _ = oracle.narrow((v * sv[None, :]).astype(np.float32))
        y[rows, :d.rows] = bf.reshape(len(rows), d.rows)
    return y


def _check(case, dev, y, acc, label):
    want = oracle_down_epilogue(case, acc)
    bad = int(np.count_nonzero(y != want))
    say(f"{label}: y vs the oracle's epilogue of the device's own sums: {bad} of {y.size} differ")
    assert bad == 0


@pytest.mark.parametrize("bits,cb", [(4, "mul1"), (3, "mcg"), (6, "3inst")])
def test_down_epilogue_bits_decode_pair(torch_cuda, bits, cb):
    """The decode path's down (k_dn): 12 tokens top-4 over 48 experts, two classes, dropped slots."""
    import exl3c4
    case = Case(seed=3100 + bits, n_tok=12, top_k=4, n_expert=48, geoms=[(512, 256), (512, 128)], bits=bits, cb=cb,
                drop=0.05)
    assert not exl3c4.is_prefill(case.T, case.n_expert)  # the decode path
    dev = Dev(case)
    h = dev.gate_up(h_rot=1)
    y = dev.down(h, h_rot=1)
    acc = dev.last_acc()
    _check(case, dev, y, acc, f"k_dn K={bits} {cb}")
    assert narrowed_ok(y, case.oracle_down(h, h_rot=1), "bf16") == 0


def test_down_epilogue_bits_single_kernel_layer_geometry(torch_cuda):
    """gate_up_down's single kernel (k_gd) at the decode layer's shapes: 8 tokens top-10 over 128 experts, K = 4."""
    import exl3c4
    case = Case(seed=3110, n_tok=8, top_k=10, n_expert=128, geoms=[(2048, 512)], bits=4, cb="mul1")
    assert case.T >= exl3c4.GD_FUSE_MIN_T and not exl3c4.is_prefill(case.T, case.n_expert)
    dev = Dev(case)
    y = dev.gate_up_down()
    assert dev.status == 0
    acc = dev.last_acc(gemm=1)
    _check(case, dev, y, acc, "k_gd K=4 mul1")


@pytest.mark.parametrize("k_gu,k_dn", [(4, 8), (8, 3)])
def test_down_epilogue_bits_single_kernel_mixed_k(torch_cuda, k_gu, k_dn):
    """k_gd with down's K apart from gate_up's (two of the 48-layer stack's pairs)."""
    case = Case(seed=3120 + k_gu + k_dn, n_tok=8, top_k=10, n_expert=128, geoms=[(2048, 512)], bits=k_gu, cb="mul1",
                dn_bits=k_dn)
    dev = Dev(case)
    y = dev.gate_up_down()
    assert dev.status == 0
    acc = dev.last_acc(gemm=1)
    _check(case, dev, y, acc, f"k_gd K_g={k_gu} K_d={k_dn}")


def test_down_epilogue_bits_prefill(torch_cuda):
    """The prefill path's down GEMM (k_dn_pf): 512 tokens top-4 over 24 experts (Zipf), two classes, drops."""
    import exl3c4
    case = Case(seed=3130, n_tok=512, top_k=4, n_expert=24, geoms=[(512, 256), (512, 128)], bits=4, cb="mul1",
                drop=0.03, routing="zipf")
    assert exl3c4.is_prefill(case.T, case.n_expert)       # the prefill path
    dev = Dev(case)
    h = dev.gate_up(h_rot=1)
    y = dev.down(h, h_rot=1)
    acc = dev.last_acc()
    _check(case, dev, y, acc, "k_dn_pf K=4 mul1")
    gd = dev.gate_up_down()
    assert np.array_equal(gd, y)
    _check(case, dev, gd, dev.last_acc(gemm=1), "gate_up_down prefill")


def test_narrowing_conversions_every_upper_half(torch_cuda):
    """The kernels' f32 -> bf16 (v_cvt_pk_bf16_f32) and f32 -> f16 against the oracle's rules over every upper half-word
    with the low halves 0, 1, 0x7FFF, 0x8000, 0x8001, 0xFFFF, and 1 M random f32 bit patterns."""
    import exl3c4
    torch = torch_cuda
    hi = np.arange(1 << 16, dtype=np.uint32) << 16
    lows = np.array([0, 1, 0x7FFF, 0x8000, 0x8001, 0xFFFF], np.uint32)
    bits = (hi[:, None] | lows[None, :]).ravel()
    rng = np.random.default_rng(3140)
    bits = np.concatenate([bits, rng.integers(0, 1 << 32, size=1 << 20, dtype=np.uint64).astype(np.uint32)])
    vals = bits.view(np.float32)
    dev_bf, dev_h = exl3c4.check_narrow(torch.from_numpy(bits.view(np.int32)).cuda().view(torch.float32))
    ref_bf, ref_h = oracle.narrow(vals)
    nan = (bits & 0x7FFFFFFF) > 0x7F800000
    say(f"narrowing: {bits.size} inputs, {int(nan.sum())} nans")
    assert np.array_equal(dev_bf, ref_bf), f"bf16: {np.count_nonzero(dev_bf != ref_bf)} differ"
    # f16: every non-nan to the bit; a nan to a nan (neither rule fixes an f16 nan's payload)
    assert np.array_equal(dev_h[~nan], ref_h[~nan]), f"f16: {np.count_nonzero(dev_h[~nan] != ref_h[~nan])} differ"
    assert np.all(((dev_h[nan] & 0x7C00) == 0x7C00) & ((dev_h[nan] & 0x03FF) != 0))
