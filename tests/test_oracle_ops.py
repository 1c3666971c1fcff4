"""The oracle's op level (or_launch: prep_gu, gate_up, down; or_gate_up_down) pinned against float64 dense products of
the pinned dense weights (tests/dense64.py) -- the reference's own device criterion, "a float64 dense
decode-and-multiply" (tests/gpu/test_exl3r4d.py:23-27), and the invariants of docs/OPS-exl3.md:303-335. CPU only.

Two tiers, both against values the oracle's op code did not compute:
  exact       the ops in float64 with no rounding: every output element within one unit in the last place of its
              format (f16 h / xr, bf16 y) at the exact value plus 8e-3 x RMS (the reference's own f16 roundings of the
              rotated input and of h, which the exact value does not have), and relative L2 <= 2e-3;
  rounded     the same float64 products with the reference's rounding points kept (kernels/exl3ref/ref.c:27-32,
              187-225: f16(x * s), f16 of the rotation, f16 h): within one ulp plus 1e-3 x RMS, and most elements
              (>= 90% of h, >= 99% of prep_gu's xr and down's y) EQUAL to the exact value rounded once.
Each tier has negative controls that plant the mistakes a restatement could make -- suh1 on the gate half, svh before
the output rotation, down scaled by its own suh instead of gate_up's dn_suh, no SiLU, a dropped rounding of the
rotated input, the class interleave e // n instead of e % n -- and shows the comparison fails on them. The
flipped-symbol control: one symbol of one expert's codes moves only that expert's rows.
"""
import numpy as np
import pytest

import dense64 as D
import oracle
from cases import Case, ordered

CASES = {
    "one-class": dict(seed=11, n_tok=4, top_k=4, n_expert=8, geoms=[(256, 128)], bits=4, cb="mul1"),
    "two-class": dict(seed=12, n_tok=6, top_k=3, n_expert=9, geoms=[(256, 256), (384, 128)], bits=4, cb="mcg",
                      drop=0.2, protect_tail=2),
    "four-class": dict(seed=13, n_tok=5, top_k=4, n_expert=11, geoms=[(256, 128), (256, 256), (128, 128), (256, 128)],
                       bits=3, cb="3inst", drop=0.15, protect_tail=1),
    "layer-shape-bf16": dict(seed=14, n_tok=3, top_k=2, n_expert=4, geoms=[(2048, 512)], bits=4, cb="mul1",
                             x_bf16=True),
}
EXACT_TOL, ROUNDED_TOL = 8e-3, 1e-3


def _ulp(v, fmt):
    p = 10 if fmt == "f16" else 7
    e = np.floor(np.log2(np.maximum(np.abs(v), 2.0 ** -14)))
    return 2.0 ** (e - p)


def _excess(got, want, fmt):
    """max over elements of (|got - want| - ulp(want)) / RMS(want)."""
    rms = np.sqrt(np.mean(want ** 2))
    return float(np.max(np.abs(got - want) - _ulp(want, fmt)) / rms)


def _rel_l2(got, want):
    return float(np.linalg.norm(got - want) / np.linalg.norm(want))


def _round(v, fmt):
    if fmt == "f16":
        return np.asarray(v).astype(np.float16).view(np.uint16)
    u = np.asarray(v, np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def _match(got_bits, want, fmt):
    return float(np.mean(ordered(got_bits) == ordered(_round(want, fmt))))


def _val(bits, fmt):
    return D.f16(bits) if fmt == "f16" else D.bf16(bits)


def _outputs(case):
    """The oracle's outputs of every op and flag on the case (what the tiers check)."""
    xr = case.oracle_prep(prefill=0)
    h = {r: case.oracle_gate_up(h_rot=r) for r in (0, 1)}
    ha = {r: case.oracle_gate_up(h_rot=r, a_rot=1, xr=xr) for r in (0, 1)}
    return dict(xr=xr, h=h, ha=ha, y0=case.oracle_down(h[0], 0), y1=case.oracle_down(h[1], 1),
                gd=case.oracle_gate_up_down())


def _checks(case, out, dense):
    """(name, got bits, want float64, fmt) of every op on the case; prep_gu only where it writes."""
    pd = dense.prep()
    m = ~np.isnan(pd)
    res = [("prep_gu", out["xr"][m], pd[m], "f16")]
    for r in (0, 1):
        res.append((f"gate_up h_rot {r}", out["h"][r], dense.gate_up(h_rot=r), "f16"))
        res.append((f"gate_up h_rot {r} a_rot 1", out["ha"][r], dense.gate_up(h_rot=r, xr=out["xr"]), "f16"))
    res.append(("down h_rot 0", out["y0"], dense.down(out["h"][0], 0), "bf16"))
    res.append(("down h_rot 1", out["y1"], dense.down(out["h"][1], 1), "bf16"))
    res.append(("gate_up_down", out["gd"], dense.gate_up_down(), "bf16"))
    return res


@pytest.fixture(scope="module", params=list(CASES))
def case_out(request):
    case = Case(**CASES[request.param])
    return request.param, case, _outputs(case)


def test_the_ops_equal_the_exact_float64_products(case_out):
    name, case, out = case_out
    for op, got, want, fmt in _checks(case, out, D.Dense(case)):
        g = _val(got, fmt)
        assert _excess(g, want, fmt) <= EXACT_TOL, f"{name} {op}: {_excess(g, want, fmt):.2e}"
        assert _rel_l2(g, want) <= 2e-3, f"{name} {op}: rel-L2 {_rel_l2(g, want):.2e}"


def test_the_ops_keep_the_reference_rounding_points(case_out):
    name, case, out = case_out
    for op, got, want, fmt in _checks(case, out, D.Dense(case, rounded=True)):
        g = _val(got, fmt)
        assert _excess(g, want, fmt) <= ROUNDED_TOL, f"{name} {op}: {_excess(g, want, fmt):.2e}"
        floor = 0.90 if op.startswith("gate_up") else 0.99
        assert _match(got, want, fmt) >= floor, f"{name} {op}: {_match(got, want, fmt):.4f} equal"


def test_dead_rows_are_zero_and_prep_leaves_them_unwritten(case_out):
    name, case, out = case_out
    dead = np.array([i >= case.off[-1] or i < case.off[0] or case.sorted_tok[i] < 0 for i in range(case.T)])
    for k in ("y0", "y1", "gd"):
        assert np.all(out[k][dead] == 0), f"{name} {k}"
    for r in (0, 1):
        assert np.all(out["h"][r][dead] == 0) and np.all(out["ha"][r][dead] == 0)
    outside = np.array([i >= case.off[-1] or i < case.off[0] for i in range(case.T)])
    pre = case.oracle_prep(prefill=0xABCD)
    assert np.all(pre[outside] == 0xABCD)                      # rows no run holds: prep_gu writes nothing there


# ------------------------------------------------------------------------------------------ negative controls
@pytest.mark.parametrize("knob,ops", [
    ("swap_suh", ("gate_up h_rot 0", "gate_up h_rot 1", "gate_up_down")),
    ("svh_before_had", ("gate_up h_rot 0", "gate_up h_rot 1", "gate_up_down")),
    ("no_silu", ("gate_up h_rot 0", "gate_up h_rot 1", "gate_up_down")),
    ("dn_own_suh", ("gate_up_down",)),
])
def test_the_exact_tier_fails_on_a_planted_mistake(knob, ops):
    case = Case(**CASES["two-class"])
    for e in range(case.n_expert):                             # gate_up_down's dn_suh unlike down's own suh
        case.gu[e].dn_suh = (case.gu[e].dn_suh.astype(np.float32) * -0.75).astype(np.float16)
    out = _outputs(case)
    for op, got, want, fmt in _checks(case, out, D.Dense(case, [knob])):
        if op in ops:
            assert _excess(_val(got, fmt), want, fmt) > 100 * EXACT_TOL, f"{knob} {op}"
    for op, got, want, fmt in _checks(case, out, D.Dense(case)):   # and the same case passes without the mistake
        assert _excess(_val(got, fmt), want, fmt) <= EXACT_TOL, op


def test_the_rounded_tier_fails_without_the_rounding_of_the_rotated_input():
    case = Case(**CASES["one-class"])
    out = _outputs(case)
    bad = {op: (got, want, fmt) for op, got, want, fmt in _checks(case, out, D.Dense(case, ["no_xr_round"],
                                                                                       rounded=True))}
    for op in ("gate_up h_rot 0", "gate_up h_rot 1"):
        got, want, fmt = bad[op]
        assert _match(got, want, fmt) < 0.80, op
    got, want, fmt = bad["gate_up_down"]
    assert _excess(_val(got, fmt), want, fmt) > ROUNDED_TOL


def test_the_class_interleave_is_pinned():
    """Tables built with expert e at class e // (E / n), entry e % (E / n) (a transposed interleave) give another
    output; the dense reference, which never uses classes, agrees only with e % n_class at entry e / n_class."""
    case = Case(**{**CASES["four-class"], "geoms": [(256, 128)] * 4, "drop": 0.0, "protect_tail": 0, "n_expert": 12})
    want = D.Dense(case).gate_up(h_rot=0)
    good = case.oracle_gate_up(h_rot=0)
    assert _excess(D.f16(good), want, "f16") <= EXACT_TOL
    per = case.n_expert // case.n_class
    cl = case.classes("gu")
    blocked = []
    for c in range(case.n_class):
        ex = [case.gu[e] for e in range(c * per, (c + 1) * per)]
        blocked.append({**cl[c], "codes": np.stack([x.codes for x in ex]), "suh": np.stack([x.suh for x in ex]),
                        "suh1": np.stack([x.suh1 for x in ex]), "svh": np.stack([x.svh for x in ex]),
                        "dn_suh": np.stack([x.dn_suh for x in ex])})
    bad = oracle.run_op(oracle.OP_GATE_UP, blocked, case.bits, case.cb, case.x, case.sorted_tok, case.off, case.top_k)
    assert _excess(D.f16(bad), want, "f16") > 100 * EXACT_TOL


@pytest.mark.parametrize("which", ["gate_up", "down", "gate_up_down"])
def test_one_flipped_symbol_moves_only_its_experts_rows(which):
    """docs/OPS-exl3.md:324-328: flip one K-bit symbol of one expert's codes; the rows of that expert change and no
    other row does (bit for bit)."""
    case = Case(**CASES["one-class"])
    live = D.Dense(case).live()
    e = max(set(live.values()), key=lambda x: sum(v == x for v in live.values()))
    rows = sorted(i for i, v in live.items() if v == e)

    def run():
        h0 = case.oracle_gate_up(h_rot=0)
        return {"gate_up": h0, "down": case.oracle_down(h0_fixed, 0), "gate_up_down": case.oracle_gate_up_down()}[which]

    h0_fixed = case.oracle_gate_up(h_rot=0)
    before = run()
    w = case.gu[e] if which != "down" else case.dn[e]
    w.codes = w.codes.copy()
    w.codes[3, 5] ^= 0x11                                       # symbol bits in row 3 (K = 4: two symbols' low bits)
    after = run()
    moved = np.any(before != after, axis=1)
    assert np.all(moved[rows]) or (which == "down" and np.any(moved[rows]))
    others = np.ones(case.T, bool)
    others[rows] = False
    assert not np.any(moved[others])
