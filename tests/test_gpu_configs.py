"""Device parity at BASELINE.json's workloads and the reference's own shapes (GPU).

  configs[2]  the decode layer: 512 experts (gate/up 2048 -> 512, down 512 -> 2048, K = 4 mul1), 8 tokens, router
              logits N(0,1) -> softmax top-10 renormalised -> stable scatter -> gate_up_down -> f32 weighted gather
              to f16, all on the device (router_topk_scatter, launch_gather), against the oracle's router, scatter,
              gate_up_down and gather: the gather to the bit on the device's y, down within one bf16 ulp on the
              device's h, and the layer output against the oracle's layer by rel-L2 <= 4e-3 (the reference's device
              criterion) and max-abs <= 2e-2 x RMS. The north star's max-abs <= 2e-3 x RMS holds for the f32
              accumulations (held in the op tests; about 1e-5 x RMS); across the op's narrowed intermediates (h f16,
              y bf16) a one-ulp flip of h, which a different summation order alone causes, is spread by down, and the
              layer output measures max-abs 9.1e-3 x RMS (rel-L2 3.3e-4).
  configs[3]  the prefill layer: 2048 tokens, Zipf(1.1) top-10 over the same 512 experts (20,480 rows, hot experts
              of many 64-row chunks), against the oracle's gate_up_down; gate_up_down == its pair, zero rows, replay,
              the checked f32 sums of sampled rows (the hottest expert's among them) within 2e-3 x RMS. And a smaller
              prefill (256 tokens over 32 experts) through every op against the oracle.
  configs[4]  one decode layer at each K in {2, 3, 6, 8} against the oracle, and the mixed-K layer (gate_up at K_g,
              down at K_d != K_g, the split chain the 48-layer stack runs).
  reference   the real per-rank geometry: hidden 2560 (20 k-blocks: a split-K whose last split holds no block),
              width 640 (5 h-blocks), and tp2's 384/256 two-class split (tests/ref/test_exl3ref.py:1103-1113,
              1147-1150); the band tops M = 16 and M = 4096, two-class and four-class (:1282-1300).
  scratch     a band's scratch, sized once at its top, takes every smaller batch (the decode split-K count grows
              as the batch shrinks) with the same bits as an exactly sized scratch, and nothing writes past it.
Every output, scratch and counter block is guarded by poisoned margins (cases.Guard), checked after each launch.
"""
import numpy as np
import pytest

import oracle
from cases import Case, Dev, bf16, f16, narrowed_ok, oracle_acc, rel_err, rel_l2
from gpuchecks import CHAIN_TOL, TOL, chain_ok, check_all, say

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def torch_cuda():
    torch = pytest.importorskip("torch")
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import exl3c4
    exl3c4.lib()          # raises if the library is not built: no fallback exists
    return torch


@pytest.fixture(scope="module")
def layer(torch_cuda):
    """The 512 experts of configs[2] / configs[3] on the device (805 MB of stored records)."""
    say("configs[2]/[3]: 512 experts 2048/512 K=4 mul1, building and uploading")
    case = Case(seed=20261013, n_tok=8, top_k=10, n_expert=512, geoms=[(2048, 512)], bits=4, cb="mul1")
    return case, Dev(case)


# ------------------------------------------------------------------------------------------ configs[2]
def test_decode_layer_configs2_with_device_routing_against_the_oracle(layer):
    import exl3c4 as ex
    case0, dev0 = layer
    torch = dev0.torch
    rng = np.random.default_rng(20261014)
    logits = rng.standard_normal((8, 512)).astype(np.float32)
    say("configs[2]: router_topk_scatter on the device")
    lg = torch.from_numpy(logits).cuda()
    ids, w = dev0.guard(8 * 10 * 4).view.view(torch.int32).view(8, 10), dev0.guard(8 * 10 * 4).view.view(
        torch.float32).view(8, 10)
    st, off = dev0.guard(80 * 4).view.view(torch.int32), dev0.guard(513 * 4).view.view(torch.int32)
    cnt, row_of = dev0.guard(512 * 4).view.view(torch.int32), dev0.guard(80 * 4).view.view(torch.int32)
    assert ex.router_topk_scatter(lg, 10, True, ids, w, st, off, cnt, row_of) == 0
    torch.cuda.synchronize()
    ids_o, w_o = oracle.router_topk(logits, 10, True)
    st_o, off_o, cnt_o, row_of_o = oracle.moe_scatter_full(ids_o, 512)
    assert np.array_equal(ids.cpu().numpy(), ids_o)
    assert np.max(np.abs(w.cpu().numpy() - w_o)) <= 2e-6
    for got, want in ((st, st_o), (off, off_o), (cnt, cnt_o), (row_of, row_of_o)):
        assert np.array_equal(got.cpu().numpy(), want)
    live = int(np.count_nonzero(cnt_o))
    say(f"configs[2]: {live} live experts; gate_up_down with the gather inside its kernel")

    case = case0.rerouted(seed=20261015, n_tok=8, top_k=10, expert_ids=ids_o)
    dev = Dev(case, share=dev0)
    assert np.array_equal(dev.sorted_tok.cpu().numpy(), st_o)
    y = dev.out(2048)
    out = dev.out(2048, rows=8)
    o = dev.gd_op(y)
    ctr = dev.guard(ex.ctr_bytes(o), fill=0)
    assert ex.launch_gather(o, dev.scratch(o), ctr.view, w, row_of, out) == 0
    torch.cuda.synchronize()
    assert int(torch.count_nonzero(ctr.view)) == 0
    dev.check_guards("configs[2] launch_gather")
    y_d, out_d = y.cpu().numpy().view(np.uint16), out.cpu().numpy().view(np.uint16)

    say("configs[2]: the oracle's layer")
    y_o = case.oracle_gate_up_down()
    out_o = oracle.moe_gather(y_o, True, w_o, row_of_o, 8, 10)
    # the gather to the bit: the oracle's gather of the device's own y with the device's weights
    assert np.array_equal(out_d, oracle.moe_gather(y_d, True, w.cpu().numpy(), row_of_o, 8, 10))
    # down on the device's own h within one bf16 ulp of the oracle's; the whole chain within the chain bar
    h1 = dev.gate_up(h_rot=1)
    assert np.array_equal(dev.down(h1, h_rot=1), y_d)              # gate_up_down == its pair
    assert narrowed_ok(y_d, case.oracle_down(h1, h_rot=1), "bf16") == 0
    assert chain_ok("configs[2] y (the whole chain)", bf16(y_d), bf16(y_o))
    err, l2 = rel_err(f16(out_d), f16(out_o)), rel_l2(f16(out_d), f16(out_o))
    say(f"configs[2] layer output vs the oracle's layer: max-abs/RMS {err:.2e}, rel-L2 {l2:.2e} "
        f"(the f32 accumulations themselves are held to 2e-3 x RMS in the op tests)")
    assert l2 <= CHAIN_TOL
    assert err <= 2e-2                                             # one-ulp flips of h and y, spread (measured 9.1e-3)


# ------------------------------------------------------------------------------------------ configs[3]
def _sample_rows(case, n_hot=24, n_other=24, seed=0):
    """Rows of the hottest expert and of others, for checks of the f32 sums at full size."""
    counts = np.diff(case.off)
    hot = int(np.argmax(counts))
    rng = np.random.default_rng(seed)
    lo, hi = int(case.off[hot]), int(case.off[hot + 1])
    rows = list(rng.choice(np.arange(lo, hi), size=min(n_hot, hi - lo), replace=False))
    live = [i for i in range(int(case.off[-1])) if case.sorted_tok[i] >= 0 and not lo <= i < hi]
    rows += list(rng.choice(live, size=min(n_other, len(live)), replace=False))
    return hot, sorted(int(r) for r in rows)


def _gu_acc_rows(case, xr, rows):
    """The oracle's gate_up f32 sums (ascending k) of the given rows only: [len(rows), N]."""
    out = []
    owner = np.searchsorted(case.off, rows, side="right") - 1
    for i, e in zip(rows, owner):
        g = case.gu[int(e)]
        what = oracle.what_rows(g.codes, g.rows, g.cols, case.bits, case.cb)
        x = f16(xr[[i]])
        W, C = g.rows // 2, g.cols
        out.append(np.concatenate([oracle_acc(x[:, :C], what[:W]), oracle_acc(x[:, C:2 * C], what[W:])], axis=1)[0])
    return np.stack(out)


def test_prefill_layer_configs3_against_the_oracle(layer):
    case0, dev0 = layer
    case = case0.rerouted(seed=20261016, n_tok=2048, top_k=10, routing="zipf")
    counts = np.diff(case.off)
    say(f"configs[3]: T={case.T}, {int(np.count_nonzero(counts))} live experts, hottest {int(counts.max())} rows")
    assert case.T == 20480 and counts.max() > 64 * 8
    dev = Dev(case, share=dev0)
    gd = dev.gate_up_down()                                      # the prefill path
    say("configs[3]: the oracle's gate_up_down")
    y_o = case.oracle_gate_up_down()
    assert chain_ok("configs[3] y (the whole chain)", bf16(gd), bf16(y_o))
    say("configs[3]: the pair; down on the device's own h against the oracle's down")
    h1 = dev.gate_up(h_rot=1)
    assert np.array_equal(dev.down(h1, h_rot=1), gd)
    bad = narrowed_ok(gd, case.oracle_down(h1, h_rot=1), "bf16")
    say(f"configs[3]: {bad} elements of down past one bf16 ulp / 1e-4 RMS")
    assert bad == 0
    dead = np.array([i >= case.off[-1] or case.sorted_tok[i] < 0 for i in range(case.T)])
    assert np.all(gd[dead] == 0)
    say("configs[3]: a replay")
    assert np.array_equal(dev.gate_up_down(), gd)
    say("configs[3]: checked f32 sums of sampled rows")
    dev.gate_up(h_rot=0)
    acc = dev.last_acc()
    hot, rows = _sample_rows(case)
    xr = case.oracle_prep(prefill=0)
    want = _gu_acc_rows(case, xr, rows)
    err = rel_err(acc[rows, :want.shape[1]], want)
    say(f"configs[3]: gate_up f32 sums of {len(rows)} rows (expert {hot} hottest): max-abs/RMS {err:.2e}")
    assert err <= TOL
    dev.check_tables()


@pytest.mark.parametrize("M", [24, 256])
def test_middle_band_against_the_oracle(layer, M):
    """The band between decode and prefill (the reference serves every M >= 17 with its prefill rows,
    kernels/exl3r4d/rows.c:255-315): M tokens, softmax top-10 over the layer's 512 experts. M = 24 (240 sorted rows)
    sits below exl3c4_prefill_min_rows and runs as the decode path's single kernel; M = 256 (2560 rows, most experts
    one to a few rows) runs the prefill path. Each: gate_up_down == its pair, the chain against the oracle's, down on the
    device's own h within one bf16 ulp, and gate_up's f32 sums of sampled rows within 2e-3 x RMS of the oracle's
    ascending sums."""
    import exl3c4
    case0, dev0 = layer
    case = case0.rerouted(seed=20261019 + M, n_tok=M, top_k=10)
    pf = exl3c4.is_prefill(case.T, case.n_expert)
    assert case.T == 10 * M and pf == (M == 256) and case.T >= exl3c4.GD_FUSE_MIN_T
    counts = np.diff(case.off)
    say(f"middle band M={M}: {int(np.count_nonzero(counts))} live experts, hottest {int(counts.max())} rows, "
        f"{'prefill' if pf else 'decode single kernel'}")
    dev = Dev(case, share=dev0)
    gd = dev.gate_up_down()
    assert dev.status == (None if pf else 0)                     # the single kernel (and no wait gave up) at M = 24
    h1 = dev.gate_up(h_rot=1)
    assert np.array_equal(dev.down(h1, h_rot=1), gd)
    assert narrowed_ok(gd, case.oracle_down(h1, h_rot=1), "bf16") == 0
    assert chain_ok(f"middle band M={M} y (the whole chain)", bf16(gd), bf16(case.oracle_gate_up_down()))
    dev.gate_up(h_rot=0)
    acc = dev.last_acc()
    hot, rows = _sample_rows(case, n_hot=8, n_other=32, seed=3)
    want = _gu_acc_rows(case, case.oracle_prep(prefill=0), rows)
    err = rel_err(acc[rows, :want.shape[1]], want)
    say(f"middle band M={M}: gate_up f32 sums of {len(rows)} rows: max-abs/RMS {err:.2e}")
    assert err <= TOL
    assert np.array_equal(dev.gate_up_down(), gd)
    dev.check_tables()


def test_prefill_multichunk_hot_experts_through_every_op(torch_cuda):
    """The prefill path at the layer's shapes against the oracle op by op: 256 tokens, Zipf top-10 over 32 experts
    (2560 rows, the hottest of several 64-row chunks)."""
    import exl3c4
    case = Case(seed=20261017, n_tok=256, top_k=10, n_expert=32, geoms=[(2048, 512)], bits=4, cb="mul1",
                routing="zipf", drop=0.01, protect_tail=3)
    assert exl3c4.is_prefill(case.T, case.n_expert) and np.diff(case.off).max() > 3 * 64
    check_all(case, "prefill 2048/512 zipf")


# ------------------------------------------------------------------------------------------ configs[4]
@pytest.mark.parametrize("bits,cb", [(2, "mul1"), (3, "mul1"), (6, "mul1"), (8, "mul1")])
def test_decode_layer_at_each_k_of_the_stack(torch_cuda, bits, cb):
    case = Case(seed=20261020 + bits, n_tok=8, top_k=10, n_expert=128, geoms=[(2048, 512)], bits=bits, cb=cb)
    dev = Dev(case)
    say(f"configs[4] layer K={bits}")
    gd = dev.gate_up_down()
    assert dev.status == 0
    h1 = dev.gate_up(h_rot=1)
    assert np.array_equal(dev.down(h1, h_rot=1), gd)
    assert narrowed_ok(gd, case.oracle_down(h1, h_rot=1), "bf16") == 0
    assert chain_ok(f"K={bits} gate_up_down", bf16(gd), bf16(case.oracle_gate_up_down()))
    dev.check_tables()


@pytest.mark.parametrize("k_gu,k_dn", [(2, 4), (6, 3), (8, 2), (3, 8)])
def test_mixed_k_layer_split_chain(torch_cuda, k_gu, k_dn):
    """A layer whose gate_up and down differ in K: gate_up(h_rot 1) at K_g, then down(h_rot 1) at K_d."""
    case = Case(seed=20261030 + 10 * k_gu + k_dn, n_tok=8, top_k=10, n_expert=128, geoms=[(2048, 512)], bits=k_gu,
                cb="mul1", dn_bits=k_dn)
    dev = Dev(case)
    say(f"configs[4] mixed layer K_g={k_gu} K_d={k_dn}")
    h1 = dev.gate_up(h_rot=1)
    h1_o = case.oracle_gate_up(h_rot=1)
    assert chain_ok("gate_up h_rot 1", f16(h1), f16(h1_o))
    y = dev.down(h1, h_rot=1)
    assert narrowed_ok(y, case.oracle_down(h1, h_rot=1), "bf16") == 0
    assert chain_ok("mixed chain", bf16(y), bf16(case.oracle_down(h1_o, h_rot=1)))
    dev.check_tables()


@pytest.mark.parametrize("k_gu,k_dn,cb,n_tok,top_k,n_expert,geom", [
    (2, 4, "mul1", 8, 10, 128, (2048, 512)),     # 80 rows: gate_up_down's single kernel at the pair (2, 4)
    (6, 3, "mul1", 8, 10, 128, (2048, 512)),
    (8, 2, "mul1", 8, 10, 128, (2048, 512)),     # the K = 8 occupancy target with a K = 2 down
    (3, 6, "mul1", 8, 10, 128, (2048, 512)),     # the four other pairs the 48-layer stack runs (bench.py run_stack:
    (4, 8, "mul1", 8, 10, 128, (2048, 512)),     # gate_up cycling {2,3,4,6,8}, down two places on), each its own
    (6, 2, "mul1", 8, 10, 128, (2048, 512)),     # instantiation of k_gd<K_g, mul1, K_d> with its own register
    (8, 3, "mul1", 8, 10, 128, (2048, 512)),     # allocation
    (2, 4, "mul1", 8, 10, 512, (2048, 512)),     # the stack's first pair over a full layer's 512 experts
    (4, 6, "mul1", 2, 10, 64, (2048, 512)),      # 20 rows: the three-kernel decode form, down at its own K
    (3, 5, "mcg", 8, 10, 128, (2048, 512)),      # a codebook without a mixed single kernel: the three-kernel form
    (5, 3, "mul1", 32, 4, 16, (512, 256)),       # 128 rows over 16 experts: the prefill GEMMs at their own K
])
def test_mixed_k_gate_up_down_in_one_launch(torch_cuda, k_gu, k_dn, cb, n_tok, top_k, n_expert, geom):
    """gate_up_down with down's K apart from gate_up's (the op's dn_bits) gives the split chain's bits: gate_up
    (h_rot 1) at K_g, then down (h_rot 1) at K_d; and the chain within the bar of the oracle's."""
    case = Case(seed=20261040 + 10 * k_gu + k_dn + n_tok, n_tok=n_tok, top_k=top_k, n_expert=n_expert, geoms=[geom],
                bits=k_gu, cb=cb, dn_bits=k_dn)
    dev = Dev(case)
    say(f"configs[4] mixed gate_up_down K_g={k_gu} K_d={k_dn} {cb} T={case.T}")
    gd = dev.gate_up_down()
    assert dev.status in (None, 0)
    h1 = dev.gate_up(h_rot=1)
    assert np.array_equal(dev.down(h1, h_rot=1), gd)
    assert chain_ok("mixed gate_up_down", bf16(gd), bf16(case.oracle_down(case.oracle_gate_up(h_rot=1), h_rot=1)))
    dev.check_tables()


# ------------------------------------------------------------------------------------------ the reference's shapes
def test_reference_geometry_tp1_2560_by_640(torch_cuda):
    check_all(Case(seed=5, n_tok=4, top_k=10, n_expert=16, geoms=[(2560, 640)], bits=4, cb="mul1"), "real tp1")


def test_reference_geometry_tp2_384_256_two_classes(torch_cuda):
    check_all(Case(seed=6, n_tok=2, top_k=10, n_expert=16, geoms=[(2560, 384), (2560, 256)], bits=4, cb="mul1"),
              "real tp2 384/256")


@pytest.mark.parametrize("M,top_k,n_expert", [(16, 10, 16), (4096, 2, 8)])
def test_band_tops_two_classes(torch_cuda, M, top_k, n_expert):
    check_all(Case(seed=4096 + M, n_tok=M, top_k=top_k, n_expert=n_expert, geoms=[(256, 256), (256, 128)], bits=4,
                   cb="mul1", drop=0.02), f"band top M={M}")


@pytest.mark.parametrize("M,top_k,n_expert", [(16, 10, 16), (4096, 2, 8)])
def test_band_tops_four_classes(torch_cuda, M, top_k, n_expert):
    check_all(Case(seed=40964 + M, n_tok=M, top_k=top_k, n_expert=n_expert,
                   geoms=[(256, 256), (256, 128), (256, 128), (256, 128)], bits=4, cb="mul1", drop=0.02),
              f"mod4 band top M={M}")


# ------------------------------------------------------------------------------------------ scratch at the band top
def test_band_top_scratch_takes_every_smaller_batch_on_the_device(torch_cuda):
    """A band of M = 80 tokens (top_k 1) sized once; batches of 1 .. 80 rows launch in it (guarded: nothing past it)
    with the bits of a launch in exactly sized scratch, including the batches that need MORE scratch than the top."""
    import exl3c4 as ex
    base = Case(seed=20261040, n_tok=80, top_k=1, n_expert=64, geoms=[(2048, 512)], bits=4, cb="mul1")
    dev0 = Dev(base)
    for n in (1, 2, 5, 16, 31, 32, 33, 50, 64, 79, 80):
        case = base.rerouted(seed=n, n_tok=n, top_k=1)
        dev = Dev(case, share=dev0)
        say(f"scratch sweep: {n} rows")
        ys = []
        for exact in (False, True):
            y = dev.out(2048)
            o = dev.gd_op(y, M=80)
            s = dev.scratch(o, exact=exact)
            assert ex.launch(o, s) == 0
            ys.append(y.cpu().numpy())
        dev.check_guards(f"scratch sweep {n}")
        assert np.array_equal(ys[0], ys[1])
        assert np.all(ys[1][[i for i in range(n) if case.sorted_tok[i] < 0]] == 0)
    assert rel_l2(bf16(ys[1].view(np.uint16)), bf16(case.oracle_gate_up_down())) <= CHAIN_TOL
