"""Device parity: libexl3c4.so's HIP kernels, called through the C-ABI, against the CPU oracle (oracle/exl3_oracle.c).

Bars: W_hat bit-exact with the reference decode; prep_gu's xr bit-exact (the same f32 butterfly and roundings); every
op's output within max-abs <= 2e-3 * RMS(output) of the oracle run on the SAME inputs (the north star's bar, fp16 in,
fp32 accumulate in the MFMA's summation order); the whole chain (gate_up_down) within relative L2 <= 4e-3 of the
oracle's chain (the reference's device criterion, tests/ref/test_exl3ref.py:336-346 -- max-abs cannot hold there:
a one-ulp f16 flip of h at an element ten times h's RMS, which summation order alone causes, is spread by the h_rot
rotation); and, to the bit, the contract's invariants: the h_rot pair equal across the flag, prep_gu -> gate_up(a_rot 1)
equal to gate_up(a_rot 0), gate_up_down equal to its pair, zero rows, prep_gu's unwritten regions, replay determinism.
"""
import numpy as np
import pytest

from cases import Case, Dev, bf16, f16, narrowed_ok, rel_err, rel_l2
from gpuchecks import acc_ok as _acc_ok, check_all as _check_all

pytestmark = pytest.mark.gpu
TOL = 2e-3
CHAIN_TOL = 4e-3


@pytest.fixture(scope="module")
def torch_cuda():
    torch = pytest.importorskip("torch")
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import exl3c4
    exl3c4.lib()          # raises if the library is not built: no fallback exists
    return torch


def _say(msg):
    print(msg, flush=True)


# ------------------------------------------------------------------------------------------ dequant, bit-exact
@pytest.mark.parametrize("bits", range(1, 9))
@pytest.mark.parametrize("cb", ["mul1", "mcg", "3inst"])
def test_dequant_is_bit_exact_against_the_oracle(torch_cuda, bits, cb):
    import exl3c4
    import exl3c4_synth as syn
    import oracle
    torch = torch_cuda
    rows, cols = 128, 256
    _say(f"dequant K={bits} {cb} [{rows}x{cols}]")
    rng = np.random.default_rng(1000 + bits)
    codes = syn.random_codes(rng, rows, cols, bits)
    rec = torch.from_numpy(exl3c4.relayout(codes, rows, cols, bits)).cuda()
    got = exl3c4.dequant(rec, rows, cols, bits, cb).cpu().numpy().view(np.uint16)
    want = oracle.what_rows(codes, rows, cols, bits, cb, f16=True)
    assert np.array_equal(got, want), f"{np.count_nonzero(got != want)} of {want.size} differ"


def test_dequant_covers_every_mul1_state_at_the_expert_geometry(torch_cuda):
    """A whole gate_up weight [1024 x 2048] at K=4 visits (nearly) all 65,536 states; every W_hat bit equal."""
    import exl3c4
    import exl3c4_synth as syn
    import oracle
    torch = torch_cuda
    rows, cols, bits = 1024, 2048, 4
    _say("dequant K=4 mul1 [1024x2048]")
    rng = np.random.default_rng(77)
    codes = syn.random_codes(rng, rows, cols, bits)
    rec = torch.from_numpy(exl3c4.relayout(codes, rows, cols, bits)).cuda()
    got = exl3c4.dequant(rec, rows, cols, bits, "mul1").cpu().numpy().view(np.uint16)
    want = oracle.what_rows(codes, rows, cols, bits, "mul1", f16=True)
    assert np.array_equal(got, want)
    table = oracle.codebook_table("mul1")
    assert np.unique(want).size == np.unique(table).size      # every value the codebook has occurs


# ------------------------------------------------------------------------------------------ the ops
SMALL = dict(n_tok=4, top_k=4, n_expert=8, geoms=[(256, 128)], bits=4, cb="mul1")


def test_ops_small_case(torch_cuda):
    _check_all(Case(seed=1, **SMALL), "small")


def test_ops_two_classes_of_different_width_with_drops_and_protected_rows(torch_cuda):
    case = Case(seed=2, n_tok=6, top_k=3, n_expert=9, geoms=[(256, 256), (384, 128)], bits=4, cb="mul1",
                drop=0.2, protect_tail=2)
    _check_all(case, "two-class")


def test_ops_bf16_input(torch_cuda):
    _check_all(Case(seed=3, x_bf16=True, **{**SMALL, "n_expert": 5}), "bf16")


@pytest.mark.parametrize("bits,cb", [(2, "mul1"), (3, "mcg"), (5, "3inst"), (6, "mul1"), (7, "mcg"), (8, "mul1")])
def test_ops_every_k_and_codebook(torch_cuda, bits, cb):
    _check_all(Case(seed=10 + bits, n_tok=3, top_k=2, n_expert=4, geoms=[(128, 128)], bits=bits, cb=cb),
               f"K={bits} {cb}")


def test_ops_four_classes(torch_cuda):
    case = Case(seed=5, n_tok=5, top_k=4, n_expert=11, geoms=[(256, 128), (256, 256), (128, 128), (256, 128)],
                bits=3, cb="mul1")
    _check_all(case, "four-class")


# ------------------------------------------------------------------------------------------ gate_up_down as one kernel
# (decode path from 32 sorted rows: gate_up units and down units in one dispatch, each down unit waiting on its row's
# counter; _check_all holds it to the bits of the gate_up -> down pair, which runs as two kernels)
FUSED = {
    "one-class": dict(seed=50, n_tok=8, top_k=6, n_expert=24, geoms=[(256, 128)], bits=4, cb="mul1", drop=0.1,
                      protect_tail=2),
    "two-class": dict(seed=51, n_tok=10, top_k=4, n_expert=12, geoms=[(256, 256), (384, 128)], bits=4, cb="mul1",
                      drop=0.2),
    "four-class-mcg": dict(seed=52, n_tok=7, top_k=8, n_expert=16,
                           geoms=[(256, 128), (256, 256), (128, 128), (256, 128)], bits=5, cb="mcg"),
    "chunks-of-many-rows": dict(seed=53, n_tok=20, top_k=2, n_expert=3, geoms=[(256, 128)], bits=3, cb="3inst",
                                x_bf16=True),
}


@pytest.mark.parametrize("name", list(FUSED))
def test_gate_up_down_as_one_kernel(torch_cuda, name):
    import exl3c4
    case = Case(**FUSED[name])
    assert case.T >= exl3c4.GD_FUSE_MIN_T and not exl3c4.is_prefill(case.T, case.n_expert)
    dev = _check_all(case, f"one kernel {name}")
    assert dev.status == 0                             # the last launch (gate_up_down) ran as one kernel


def test_gate_up_down_as_one_kernel_at_the_layer_geometry(torch_cuda):
    """The decode layer's expert shapes (gate/up 2048 -> 512, down 512 -> 2048, K=4), 8 tokens top-10 over 128 experts:
    the single kernel's bits equal the pair's, and replays agree."""
    case = Case(seed=54, n_tok=8, top_k=10, n_expert=128, geoms=[(2048, 512)], bits=4, cb="mul1")
    dev = Dev(case)
    _say("one kernel, layer geometry")
    gd = dev.gate_up_down()
    assert dev.status == 0
    y = dev.down(dev.gate_up(h_rot=1), h_rot=1)
    assert np.array_equal(gd, y)
    for _ in range(3):
        assert np.array_equal(dev.gate_up_down(), gd)


# ------------------------------------------------------------------------------------------ the prefill path
# (from exl3c4_prefill_min_rows(n_expert) sorted rows: chunks of up to 112 rows where the launch's K are at most 4, 96
# above, a plan, the rotation into scratch, the prefill GEMMs)
def test_prefill_path_two_classes_several_chunks_with_drops(torch_cuda):
    """Runs of 126, 53, 111 and 63 rows at K = 4 (chunks of up to 112 rows): 126 cut into a full chunk of seven row
    tiles (rows past 64 read their sorted_tok from the second register) and a short one, 111 one chunk of seven
    tiles, the others one chunk of four."""
    case = Case(seed=40, n_tok=200, top_k=2, n_expert=4, geoms=[(256, 256), (384, 128)], bits=4, cb="mul1",
                drop=0.1, protect_tail=2, routing="zipf")
    import exl3c4
    assert exl3c4.is_prefill(case.T, case.n_expert) and np.diff(case.off).max() > 96
    _check_all(case, "prefill two-class")


@pytest.mark.parametrize("bits,dn_bits", [(4, 4), (6, 6), (4, 6)])
def test_prefill_chunks_by_k(torch_cuda, bits, dn_bits):
    """A run of 250 rows beside one of 50 (top_k 1, 300 sorted rows): at K 4 / 4 the plan cuts it into chunks of 112
    rows (seven row tiles), at 6 / 6 and at gate_up 4 with down 6 (one launch, down's K apart) into chunks of 96 (six:
    the kernels at K > 4 hold no seventh tile); every op of the case against the oracle."""
    import exl3c4
    ids = np.random.default_rng(96).permutation(np.array([0] * 250 + [1] * 50, dtype=np.int32))[:, None]
    case = Case(seed=96, n_tok=300, top_k=1, n_expert=2, geoms=[(256, 128)], bits=bits, cb="mul1", expert_ids=ids,
                dn_bits=dn_bits)
    assert case.T == 300 and exl3c4.is_prefill(case.T, case.n_expert)
    if bits == dn_bits:
        _check_all(case, f"prefill chunks K {bits}")
        return
    from gpuchecks import chain_ok
    _say(f"prefill chunks K {bits} / {dn_bits}")                # one launch of mixed K: its split chain's bits
    dev = Dev(case)
    gd = dev.gate_up_down()
    h1 = dev.gate_up(h_rot=1)
    h1_o = case.oracle_gate_up(h_rot=1)
    assert chain_ok("gate_up h_rot 1", f16(h1), f16(h1_o))
    assert np.array_equal(dev.down(h1, h_rot=1), gd)
    assert narrowed_ok(gd, case.oracle_down(h1, h_rot=1), "bf16") == 0
    assert chain_ok("mixed chain", bf16(gd), bf16(case.oracle_down(h1_o, h_rot=1)))
    dev.check_tables()


def test_prefill_path_four_classes_mcg(torch_cuda):
    case = Case(seed=41, n_tok=64, top_k=2, n_expert=8, geoms=[(256, 128), (256, 256), (128, 128), (256, 128)],
                bits=5, cb="mcg")
    _check_all(case, "prefill four-class")


@pytest.mark.parametrize("n_expert", [575, 576, 600])
def test_owner_search_on_both_sides_of_its_one_round_form(torch_cuda, n_expert):
    """The rotation kernels' owner search (k_prep's and k_rot's) holds the run offsets of up to 575 experts in one round
    of loads and reads the owner's run bounds out of its registers; from 576 experts it loops over the offsets and
    loads the bounds again. 600 sorted rows over 575, 576 and 600 experts (the prefill path: T >= 7/8 n_expert), with
    dropped slots, through every op against the oracle."""
    import exl3c4
    case = Case(seed=45 + n_expert, n_tok=150, top_k=4, n_expert=n_expert, geoms=[(256, 128)], bits=4, cb="mul1",
                drop=0.05)
    assert exl3c4.is_prefill(case.T, case.n_expert)
    _check_all(case, f"owner search, {n_expert} experts")


def test_prefill_plan_with_offsets_that_do_not_ascend(torch_cuda):
    """The plan's other record of the held rows. Offsets [100, 20, 50, 120, 160] over 4 experts (160 sorted rows):
    expert 0's run [100, max(20, 100)) is empty, experts 1-3 hold [20, 50), [50, 120), [120, 160) once each, and no
    run holds [0, 20). The held rows are then no single span from off[0], so the plan writes each row's owner and the
    dead-row zeroing reads it (ascending offsets take the span instead). y equals the oracle's chain on the same
    offsets (kernels/exl3r4d/launch.c:14-15 clamps the runs alike), the rows no run holds are zero, and a replay
    writes the same bits."""
    import exl3c4
    from gpuchecks import chain_ok
    case = Case(seed=91, n_tok=40, top_k=4, n_expert=4, geoms=[(256, 128)], bits=4, cb="mul1")
    assert case.T == 160 and exl3c4.is_prefill(case.T, case.n_expert)
    case.off = np.array([100, 20, 50, 120, 160], dtype=case.off.dtype)
    _say("prefill plan, offsets that do not ascend")
    dev = Dev(case)
    gd = dev.gate_up_down()
    assert chain_ok("gate_up_down", bf16(gd), bf16(case.oracle_gate_up_down()))
    dead = np.array([i < 20 or case.sorted_tok[i] < 0 for i in range(case.T)])
    assert dead[:20].all() and not dead.all()
    assert np.all(gd[dead] == 0)
    assert np.any(gd[~dead] != 0)
    assert np.array_equal(dev.gate_up_down(), gd)
    dev.check_tables()


def test_prefill_plan_past_its_register_form(torch_cuda):
    """1040 experts: past the 4 x 256 experts the rotation launch's planning workgroup holds in its threads, so the
    plan takes its general form (blocks of 256 experts, the entries read back); 960 sorted rows, every op against
    the oracle."""
    import exl3c4
    case = Case(seed=93, n_tok=240, top_k=4, n_expert=1040, geoms=[(256, 128)], bits=4, cb="mul1", drop=0.05)
    assert exl3c4.is_prefill(case.T, case.n_expert)
    _check_all(case, "prefill 1040 experts")


XCD_CROWD = [1] * 26 + [1042, 2577, 1375, 2556]      # rows an expert, top_k 1: 7,576 sorted rows


def test_prefill_xcd_ranges_hold_every_chunk_of_a_crowded_range(torch_cuda):
    """26 one-row experts, then 4 experts of 1,042-2,577 rows (top_k 1): the plan deals down's chunks to the XCDs by
    cost, and the range of the one-row chunks holds 26 of them, one more than a bound from max_chunks alone gives
    an XCD (25), whose last chunk's rows of y would go uncomputed. The bound counts the tiles the launch can hold
    (T / 16 + n_expert, the plan dropping chunks past that budget), and every op of the case meets the oracle."""
    import exl3c4
    ids = np.repeat(np.arange(len(XCD_CROWD), dtype=np.int32), XCD_CROWD)
    ids = np.random.default_rng(95).permutation(ids)[:, None]
    case = Case(seed=95, n_tok=ids.shape[0], top_k=1, n_expert=len(XCD_CROWD), geoms=[(256, 128)], bits=4,
                cb="mul1", expert_ids=ids)
    assert case.T == 7576 and exl3c4.is_prefill(case.T, case.n_expert)
    _check_all(case, "prefill crowded XCD range")


def test_prefill_units_dealt_by_the_xcd_cursors(torch_cuda):
    """Two experts of 1,900 and 148 rows (top_k 1, 2,048 sorted rows, 22 chunks): each XCD's range holds a few
    chunks' units, fewer than the round a cursor deals, so every unit of gate_up's GEMM goes out through the XCDs'
    cursors, and the XCDs whose ranges are spent (or empty) take units from the others (down's units keep their
    slots). Every op of the case meets the oracle, and a replay writes the same bits (each unit handed out once,
    wherever it ran)."""
    import exl3c4
    ids = np.array([0] * 1900 + [1] * 148, dtype=np.int32)
    ids = np.random.default_rng(99).permutation(ids)[:, None]
    case = Case(seed=99, n_tok=ids.shape[0], top_k=1, n_expert=2, geoms=[(256, 128)], bits=4, cb="mul1",
                expert_ids=ids)
    assert case.T == 2048 and exl3c4.is_prefill(case.T, case.n_expert)
    _check_all(case, "prefill units by cursors")


@pytest.mark.parametrize("n_tok,top_k", [(6, 2), (96, 4)])
def test_rotations_give_exact_zeros_the_reference_sign(torch_cuda, n_tok, top_k):
    """x of small integers and suh, suh1 of +-1: many rotated values are exact zeros (sums that cancel). The
    reference's stages are exact-sign a + b, a - b (common/exl3_decode.c:172-189; its device form
    kernels/exl3r4d/exl3r4d_common.hip.h:178-182 likewise), so such a zero is +0; the device's one-instruction DPP
    stages leave half the lanes negated and undo it by a final fma with +0, which makes every zero +0: prep_gu's xr
    equals the oracle's to the bit. Token 0's x is all zeros: its blocks rotate to +0 throughout, where the oracle's
    butterflies on the signed zeros of x su leave -0 at some outputs -- the same values, the one place the sign bits
    differ; so do the h_rot rotations of its rows' h (zero too), on the decode path (6 tokens) and the prefill path
    (96 tokens, 384 sorted rows), while every other row's h_rot output is down's first step on h to the bit."""
    import exl3c4
    case = Case(seed=97, n_tok=n_tok, top_k=top_k, n_expert=4, geoms=[(256, 128)], bits=4, cb="mul1")
    assert exl3c4.is_prefill(case.T, case.n_expert) == (n_tok > 6)
    rng = np.random.default_rng(98)
    x = rng.integers(-2, 3, size=(n_tok, 256)).astype(np.float16)
    x[0] = 0
    case.x = x.view(np.uint16)
    for g in case.gu:
        g.suh = (rng.integers(0, 2, 256) * 2 - 1).astype(np.float16)
        g.suh1 = (rng.integers(0, 2, 256) * 2 - 1).astype(np.float16)
    _say(f"rotation zero signs, {n_tok} tokens")
    dev = Dev(case)
    xr_d, xr_o = dev.prep(), case.oracle_prep()
    st = case.sorted_tok
    held = np.array([case.off[0] <= i < case.off[-1] and st[i] >= 0 for i in range(case.T)])
    zero_tok = held & (st // top_k == 0)
    rest = ~zero_tok
    assert zero_tok.any() and rest.any()
    assert np.array_equal(xr_d[rest], xr_o[rest]), f"{np.count_nonzero(xr_d[rest] != xr_o[rest])} elements differ"
    n_zero = int(np.count_nonzero(xr_o[rest & held] == 0))
    _say(f"  {n_zero} exact +0 outputs among {xr_o[rest & held].size} held values")
    assert n_zero >= xr_o[rest & held].size // 100
    assert np.all(xr_d[zero_tok] == 0)                                  # +0 throughout
    assert np.all(f16(xr_o[zero_tok]) == 0) and np.any(xr_o[zero_tok] == 0x8000)

    h0 = dev.gate_up(h_rot=0)
    h1, want = dev.gate_up(h_rot=1), case.h_rot_of(h0)
    assert np.all(f16(h0[zero_tok]) == 0)
    assert np.array_equal(h1[rest], want[rest])
    assert np.all(h1[zero_tok] == 0) and np.all(f16(want[zero_tok]) == 0)


def test_prefill_path_bf16_3inst(torch_cuda):
    _check_all(Case(seed=42, n_tok=64, top_k=1, n_expert=2, geoms=[(256, 128)], bits=3, cb="3inst", x_bf16=True),
               "prefill bf16")


@pytest.mark.parametrize("bits", [3, 4, 5])
@pytest.mark.parametrize("m", [1, 4, 16])
def test_single_routed_expert_at_the_baseline_geometry(torch_cuda, bits, m):
    """one SwiGLU expert, gate/up 2048 -> 512, down 512 -> 2048, m tokens, top_k = 1."""
    case = Case(seed=20 + bits * 100 + m, n_tok=m, top_k=1, n_expert=1, geoms=[(2048, 512)], bits=bits, cb="mul1")
    dev = Dev(case)
    _say(f"single expert K={bits} m={m}")
    gd = dev.gate_up_down()
    assert rel_l2(bf16(gd), bf16(case.oracle_gate_up_down())) <= CHAIN_TOL
    h0 = dev.gate_up(h_rot=0)
    xr_o = case.oracle_prep()
    assert _acc_ok(dev.last_acc(), case.oracle_gu_acc(xr_o), case, "gu")
    assert narrowed_ok(h0, case.oracle_gate_up(h_rot=0), "f16") == 0
    h1 = dev.gate_up(h_rot=1)
    assert np.array_equal(h1, case.h_rot_of(h0))
    assert narrowed_ok(gd, case.oracle_down(h1, h_rot=1), "bf16") == 0


# ------------------------------------------------------------------------------------------ the caller's counter block
def test_gate_up_down_with_a_counter_block_leaves_it_zero_and_gives_the_same_bits(torch_cuda):
    """exl3c4_launch_ctr: gate_up_down's single kernel takes its counters from a block the caller zeroed once; after
    every launch the block is zero again (each row's last down unit zeroes the row's counters) and the output is the
    bits of exl3c4_launch, which zeroes counters in scratch itself. Several launches in a row on one block, with
    different routing draws and row counts."""
    import exl3c4 as ex
    torch = torch_cuda
    ctr = None
    for seed, n_tok, top_k, n_expert in ((70, 8, 10, 128), (71, 6, 8, 40), (72, 8, 10, 128), (73, 4, 8, 12)):
        case = Case(seed=seed, n_tok=n_tok, top_k=top_k, n_expert=n_expert, geoms=[(512, 256)], bits=4, cb="mul1",
                    drop=0.05)
        dev = Dev(case)
        want = dev.gate_up_down()
        assert dev.status == 0
        N = max(d["rows"] for d in dev.tabs["dn"])
        y = dev.out(N, fill=0x1234)
        dn = [ex.make_class(d["rows"], d["cols"], codes=d["codes"], svh=d["svh"]) for d in dev.tabs["dn"]]
        o = ex.make_op(ex.GU_DN, case.bits, case.cb, dev.cls("gu"), dev.x, dev.sorted_tok, dev.off, y, 8, case.top_k,
                       dn=dn)
        assert case.T >= ex.GD_FUSE_MIN_T and ex.ctr_bytes(o) > 0
        if ctr is None:
            ctr = dev.guard(max(ex.ctr_bytes(o), 256), fill=0).view
        s = dev.scratch(o)
        assert ex.launch_ctr(o, s, ctr) == 0
        torch.cuda.synchronize()
        assert int(torch.count_nonzero(ctr)) == 0, f"seed {seed}: the counter block is not zero after the launch"
        assert np.array_equal(y.cpu().numpy().view(np.uint16), want)
        dev.check_guards(f"launch_ctr seed {seed}")


# ------------------------------------------------------------------------------------------ the gather in the op's kernel
@pytest.mark.parametrize("seed,n_tok,top_k,n_expert,geoms,drop,empty", [
    (80, 8, 10, 128, [(512, 256)], 0.05, False),                # one kernel, dropped pairs
    (81, 6, 8, 40, [(512, 256), (256, 128)], 0.0, False),       # two classes: the narrower one's blocks are zero
    (82, 8, 10, 128, [(512, 256)], 0.0, True),                  # a token whose slots all drop
    (83, 5, 8, 12, [(256, 128)], 0.1, False),                   # few experts: chunks of several rows
    (84, 2, 8, 12, [(256, 128)], 0.0, False),                   # T = 16: two kernels, then the gather's own
    (85, 1, 2, 4, [(256, 128), (512, 256)], 0.0, False),       # T = 2: the smallest h formed by the epilogue kernel
    (86, 3, 10, 16, [(512, 256)], 0.2, False),                  # T = 30, the largest below the one-kernel form
])
def test_launch_gather_gives_the_bits_of_the_launch_and_the_gather(torch_cuda, seed, n_tok, top_k, n_expert, geoms,
                                                                   drop, empty):
    """exl3c4_launch_gather: y and out bit for bit those of exl3c4_launch followed by exl3c4_moe_gather, out those of
    the oracle's gather over the oracle's y; the counter block zero after each of two launches in a row (the second
    with fewer tokens)."""
    import exl3c4 as ex
    import oracle
    torch = torch_cuda
    ctr = None
    for rep, nt in enumerate((n_tok, max(1, n_tok - 3))):
        ids = None
        if empty:
            rng0 = np.random.default_rng(seed)
            ids = np.stack([rng0.permutation(n_expert)[:top_k] for _ in range(nt)]).astype(np.int32)
            ids[nt // 2] = -1
        case = Case(seed=seed + 100 * rep, n_tok=nt, top_k=top_k, n_expert=n_expert, geoms=geoms, bits=4, cb="mul1",
                    drop=drop, expert_ids=ids)
        dev = Dev(case)
        want_y = dev.gate_up_down()
        assert dev.status in (0, None)                            # None: fewer rows than the one-kernel path takes
        N = max(d["rows"] for d in dev.tabs["dn"])
        dn = [ex.make_class(d["rows"], d["cols"], codes=d["codes"], svh=d["svh"]) for d in dev.tabs["dn"]]
        _, _, _, row_of = oracle.moe_scatter_full(case.ids, n_expert)
        w = np.random.default_rng(seed + 7).random((nt, top_k)).astype(np.float32)
        wt, rt = torch.from_numpy(w).cuda(), torch.from_numpy(row_of).cuda()
        outs, ys = [], []
        if ctr is None:                                           # one guarded counter block for both launches
            ctr = dev.guard(1 << 16, fill=0)
        for fused in (True, False):
            y = dev.out(N, fill=0x1234)
            out = dev.out(N, fill=0x1234, rows=nt)
            o = ex.make_op(ex.GU_DN, case.bits, case.cb, dev.cls("gu"), dev.x, dev.sorted_tok, dev.off, y, nt,
                           case.top_k, dn=dn)
            s = dev.scratch(o)
            print(f"launch_gather seed {seed} rep {rep} T {case.T} fused {fused}", flush=True)
            if fused:
                assert ctr.n >= ex.ctr_bytes(o)
                assert ex.launch_gather(o, s, ctr.view, wt, rt, out) == 0
            else:
                assert ex.launch(o, s) == 0
                assert ex.moe_gather(y, True, wt, rt, out) == 0
            torch.cuda.synchronize()
            ys.append(y.cpu().numpy().view(np.uint16))
            outs.append(out.cpu().numpy().view(np.uint16))
        assert int(torch.count_nonzero(ctr.view)) == 0, "the counter block is not zero after the launch"
        assert ctr.ok() and np.array_equal(ys[0], want_y) and np.array_equal(ys[1], want_y)
        assert np.array_equal(outs[0], outs[1])
        assert np.array_equal(outs[0], oracle.moe_gather(want_y, True, w, row_of, nt, top_k))


def test_launch_gather_with_rows_past_t_leaves_the_counter_block_good(torch_cuda):
    """row_of entries past T -- the scatter's rows of 80 pairs, the op launched over its first 70 -- name no row of
    this launch: the fused gather counts a token's slots by the same predicate (0 <= row < T) as it sums them and as
    its empty-token pass reads them, so every token completes and its counters return to zero. A second launch on the
    same counter block (all 80 rows, in contract) then gives the bits of exl3c4_launch + exl3c4_moe_gather."""
    import exl3c4 as ex
    import oracle
    torch = torch_cuda
    case = Case(seed=87, n_tok=8, top_k=10, n_expert=128, geoms=[(512, 256)], bits=4, cb="mul1")
    dev = Dev(case)
    N = max(d["rows"] for d in dev.tabs["dn"])
    _, _, _, row_of = oracle.moe_scatter_full(case.ids, case.n_expert)
    rt = torch.from_numpy(row_of).cuda()
    w = np.random.default_rng(88).random((case.n_tok, case.top_k)).astype(np.float32)
    wt = torch.from_numpy(w).cuda()
    ctr = dev.guard(1 << 16, fill=0)
    T_short = 70
    assert case.T == 80 and np.any(row_of >= T_short) and T_short >= ex.GD_FUSE_MIN_T
    y = dev.out(N, rows=T_short)
    out = dev.out(N, rows=case.n_tok)
    o = dev.gd_op(y)
    assert o.T == T_short
    print(f"launch_gather over {T_short} of {case.T} rows", flush=True)
    assert ex.launch_gather(o, dev.scratch(o), ctr.view, wt, rt, out) == 0
    torch.cuda.synchronize()
    assert int(torch.count_nonzero(ctr.view)) == 0, "rows past T left counters behind"
    print("launch_gather over all rows, same counter block", flush=True)
    y2, out2 = dev.out(N), dev.out(N, rows=case.n_tok)
    o2 = dev.gd_op(y2)
    assert ex.launch_gather(o2, dev.scratch(o2), ctr.view, wt, rt, out2) == 0
    y3, out3 = dev.out(N), dev.out(N, rows=case.n_tok)
    o3 = dev.gd_op(y3)
    assert ex.launch(o3, dev.scratch(o3)) == 0
    assert ex.moe_gather(y3, True, wt, rt, out3) == 0
    torch.cuda.synchronize()
    assert torch.equal(y2, y3) and torch.equal(out2, out3)
    assert int(torch.count_nonzero(ctr.view)) == 0
    dev.check_guards("launch_gather with rows past T")
