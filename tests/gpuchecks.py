"""gpuchecks.py -- the device-vs-oracle checks every op-level GPU test runs (shared by the test modules).

check_all runs each op of a case on the device through the C-ABI and holds it to the bars of tests/test_gpu_parity.py:
W_hat-level bits where the arithmetic is the same (prep_gu, the h_rot and a_rot equalities, gate_up_down == its pair,
zero rows, replays), the f32 accumulations within max-abs 2e-3 x RMS of the oracle's ascending sums, narrowed outputs
within one ulp (or 1e-4 x RMS) of the oracle's, and chains within relative L2 4e-3 -- printing max-abs / RMS of every
chain beside it (the north star's measure).
"""
import numpy as np

from cases import Dev, bf16, f16, narrowed_ok, rel_err, rel_l2

TOL = 2e-3
CHAIN_TOL = 4e-3


def say(msg):
    print(msg, flush=True)


def chain_ok(label, got, want):
    """relative L2 <= CHAIN_TOL; prints it and max-abs / RMS."""
    r, m = rel_l2(got, want), rel_err(got, want)
    say(f"  {label}: rel-L2 {r:.2e}, max-abs/RMS {m:.2e}")
    return r <= CHAIN_TOL


def acc_ok(got, want, case, which):
    """The north star's bar on the f32 accumulations themselves: max-abs <= 2e-3 x RMS over each live row's own
    columns (a narrower class's row has fewer)."""
    g, w = [], []
    for e, rows in case.live_rows().items():
        n = (case.gu if which == "gu" else case.dn)[e].rows
        g.append(got[rows, :n].ravel())
        w.append(want[rows, :n].ravel())
    return rel_err(np.concatenate(g), np.concatenate(w)) <= TOL


def check_all(case, label):
    dev = Dev(case)
    say(f"{label}: prep_gu")
    xr_d = dev.prep()
    xr_o = case.oracle_prep()
    assert np.array_equal(xr_d, xr_o), f"prep_gu: {np.count_nonzero(xr_d != xr_o)} elements differ"

    say(f"{label}: gate_up h_rot 0 / 1, a_rot 0 / 1")
    h0 = dev.gate_up(h_rot=0)
    N = max(g.rows for g in case.gu)
    assert acc_ok(dev.last_acc()[:, :N], case.oracle_gu_acc(xr_o), case, "gu")
    h0_o = case.oracle_gate_up(h_rot=0)
    assert narrowed_ok(h0, h0_o, "f16") == 0
    assert chain_ok("gate_up h_rot 0", f16(h0), f16(h0_o))
    h1 = dev.gate_up(h_rot=1)
    assert np.array_equal(h1, case.h_rot_of(h0))        # h_rot = 1 is down's first step on its own h, to the bit
    assert chain_ok("gate_up h_rot 1", f16(h1), f16(case.oracle_gate_up(h_rot=1)))
    xr_t = dev.torch.from_numpy(xr_d.view(np.int16)).cuda()
    assert np.array_equal(dev.gate_up(h_rot=0, a_rot=1, xr=xr_t), h0)          # prep_gu -> gate_up(a_rot 1): same bits
    assert np.array_equal(dev.gate_up(h_rot=1, a_rot=1, xr=xr_t), h1)

    say(f"{label}: down h_rot 0 / 1, gate_up_down")
    y0 = dev.down(h0, h_rot=0)                         # the oracle's down on the DEVICE's h: isolates down
    Nd = max(d.rows for d in case.dn)
    assert acc_ok(dev.last_acc()[:, :Nd], case.oracle_dn_acc(h0, h_rot=0), case, "dn")
    y0_o = case.oracle_down(h0, h_rot=0)
    assert narrowed_ok(y0, y0_o, "bf16") == 0
    assert chain_ok("down h_rot 0", bf16(y0), bf16(y0_o))
    y1 = dev.down(h1, h_rot=1)
    assert np.array_equal(y1, y0)                      # the pair's bits do not depend on h_rot
    gd = dev.gate_up_down()
    assert np.array_equal(gd, y1)                      # gate_up_down is its pair, to the bit
    assert chain_ok("gate_up_down", bf16(gd), bf16(case.oracle_gate_up_down()))
    assert narrowed_ok(gd, case.oracle_down(h1, h_rot=1), "bf16") == 0

    # zero rows: dropped slots, rows past the live count (whatever sorted_tok holds there), outside the runs
    T, n_live = case.T, int(case.off[-1])
    dead = np.array([i >= n_live or i < case.off[0] or case.sorted_tok[i] < 0 for i in range(T)])
    for out in (h0, h1, y0, gd):
        assert np.all(out[dead] == 0)
    # determinism: a replay writes the same bytes; no launch changed a weight table
    assert np.array_equal(dev.gate_up_down(), gd)
    dev.check_tables()
    return dev
