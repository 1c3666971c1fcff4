"""cases.py -- random routed-expert cases shared by the oracle-level and the device parity tests.

A case is numpy data only (canonical planes, scales, routing, activations). `oracle_*` run the CPU restatement;
`Dev` uploads the case (codes through the library's own relayout, as a loader would) and runs the device ops through
the C-ABI (radiance-exl3_amd/exl3c4.py). Every device output, scratch and counter block sits between two poisoned
256-byte margins, and every launch is followed by a check that the margins and the op's inputs are unchanged (the
reference harness's redzones, tests/ref/exl3ref_run.cpp:30-33, 56-57).
"""
from __future__ import annotations

import numpy as np

import exl3c4_synth as syn
import oracle

oracle.set_threads(oracle.default_threads())      # the checker's experts over the host's cores (same bits)
MARGIN = 256
POISON = 0xA5


class Expert:
    def __init__(self, rng, rows, cols, bits, stacked, dn_width=None, suh_mag=1.0, svh_mag=None):
        self.rows, self.cols, self.bits = rows, cols, bits
        self.codes = syn.random_codes(rng, rows, cols, bits)
        self.suh = syn.varied_scales(rng, cols, suh_mag)
        self.suh1 = syn.varied_scales(rng, cols, suh_mag) if stacked else None
        self.svh = syn.varied_scales(rng, rows, svh_mag if svh_mag else 1.0 / np.sqrt(cols))
        self.dn_suh = None


class Case:
    """n_expert experts of n_class classes: gate_up [2W_c, H_c] and down [H_c, W_c] per expert, class c = e % n_class."""

    def __init__(self, seed, n_tok, top_k, n_expert, geoms, bits, cb, drop=0.0, protect_tail=0, x_bf16=False,
                 routing="uniform", expert_ids=None, dn_bits=None):
        rng = np.random.default_rng(seed)
        self.rng = rng
        self.n_expert, self.bits, self.cb = n_expert, bits, cb
        self.dn_bits = bits if dn_bits is None else dn_bits    # down's K (a layer of mixed K: gate_up then down)
        self.n_class = len(geoms)
        self.geoms = geoms                                  # per class (H, W): hidden, width
        self.gu, self.dn = [], []
        for e in range(n_expert):
            H, W = geoms[e % self.n_class]
            g = Expert(rng, 2 * W, H, bits, True)
            d = Expert(rng, H, W, self.dn_bits, False)
            g.dn_suh = d.suh                                # down's suh of the same expert
            self.gu.append(g)
            self.dn.append(d)
        self.route(rng, n_tok, top_k, drop, protect_tail, x_bf16, routing, expert_ids)

    def rerouted(self, seed, n_tok, top_k, drop=0.0, protect_tail=0, x_bf16=False, routing="uniform",
                 expert_ids=None):
        """The same experts under another routing draw and batch (a shallow copy: the experts are shared)."""
        c = object.__new__(Case)
        c.__dict__.update(self.__dict__)
        c.rng = np.random.default_rng(seed)
        c.route(c.rng, n_tok, top_k, drop, protect_tail, x_bf16, routing, expert_ids)
        return c

    def route(self, rng, n_tok, top_k, drop, protect_tail, x_bf16, routing, expert_ids):
        n_expert, geoms = self.n_expert, self.geoms
        self.n_tok, self.top_k = n_tok, top_k
        Hmax = max(h for h, _ in geoms)
        self.x_bf16 = x_bf16
        x = rng.standard_normal((n_tok, Hmax)).astype(np.float32)
        if x_bf16:
            self.x = (x.view(np.uint32) >> 16).astype(np.uint16)          # bf16 bits (truncation: any bits are fine)
        else:
            self.x = x.astype(np.float16).view(np.uint16)
        if expert_ids is not None:                          # a given routing (the device router's, say)
            ids, w = np.asarray(expert_ids, np.int32), None
        elif routing == "zipf":
            ids, w = syn.zipf_topk(rng, n_tok, n_expert, top_k)
        else:
            ids, w = syn.router_topk(rng.standard_normal((n_tok, n_expert)), top_k)
        if drop:
            kill = rng.random(ids.shape) < drop
            ids = np.where(kill, -1, ids).astype(np.int32)
        self.ids, self.w = ids, w
        st, off = syn.moe_scatter(ids, n_expert)
        if protect_tail:
            # rows past the live count that hold valid flat indices (a `protect` sort): the ops must zero them
            n_live = int(off[-1])
            take = min(protect_tail, st.size - n_live)
            st[n_live:n_live + take] = np.arange(take)
        self.sorted_tok, self.off = st, off
        self.T = st.size

    # ------------------------------------------------------------------ class tables (numpy, stacked)
    def classes(self, which):
        """Class c's stacked tables (experts e % n_class == c at entry e / n_class), cached by the identity of the
        experts' arrays (a test that replaces one gets fresh tables)."""
        experts = self.gu if which == "gu" else self.dn
        key = (which, tuple((id(x.codes), id(x.suh), id(x.svh), id(getattr(x, "suh1", None)),
                             id(getattr(x, "dn_suh", None))) for x in experts))
        cache = self.__dict__.setdefault("_cls_cache", {})
        hit = cache.get(which)
        if hit is not None and hit[0] == key:
            return hit[1]
        out = []
        for c in range(self.n_class):
            ex = [experts[e] for e in range(c, self.n_expert, self.n_class)]
            d = {"rows": ex[0].rows, "cols": ex[0].cols,
                 "codes": np.stack([x.codes for x in ex]), "suh": np.stack([x.suh for x in ex]),
                 "svh": np.stack([x.svh for x in ex])}
            if which == "gu":
                d["suh1"] = np.stack([x.suh1 for x in ex])
                d["dn_suh"] = np.stack([x.dn_suh for x in ex])
            out.append(d)
        cache[which] = (key, out)                       # one set of tables a side at a time (large cases)
        return out

    # ------------------------------------------------------------------ the oracle
    def oracle_prep(self, prefill=0xFFFF):
        cl = self.classes("gu")
        y = np.full((self.T, 2 * max(c["cols"] for c in cl)), prefill, np.uint16)
        return oracle.run_op(oracle.OP_PREP_GU, cl, self.bits, self.cb, self.x, self.sorted_tok, self.off,
                             self.top_k, x_bf16=self.x_bf16, y=y)

    def oracle_gate_up(self, h_rot=0, a_rot=0, xr=None):
        x = xr if a_rot else self.x
        return oracle.run_op(oracle.OP_GATE_UP, self.classes("gu"), self.bits, self.cb, x, self.sorted_tok, self.off,
                             self.top_k, h_rot=h_rot, a_rot=a_rot, x_bf16=self.x_bf16 and not a_rot)

    def oracle_down(self, h, h_rot=0):
        return oracle.run_op(oracle.OP_DOWN, self.classes("dn"), self.dn_bits, self.cb, h, self.sorted_tok, self.off,
                             self.top_k, h_rot=h_rot)

    def h_rot_of(self, h0):
        """What gate_up's h_rot = 1 output must be, to the bit, given its h_rot = 0 output h0: down's first step
        f16(had(f16(h0 * dn_suh))) on each live row (docs/OPS-exl3.md:120-123), zeros elsewhere."""
        out = np.zeros_like(h0)
        for i in range(self.T):
            if i < self.off[0] or i >= self.off[-1] or self.sorted_tok[i] < 0:
                continue
            e = int(np.searchsorted(self.off, i, side="right") - 1)
            g = self.gu[e]
            W = g.rows // 2
            xr = oracle.prologue(f16(h0[i, :W]), g.dn_suh)
            out[i, :W] = xr.astype(np.float16).view(np.uint16)
        return out

    def live_rows(self):
        """{expert: [rows]} of the rows an op computes: inside the runs, sorted_tok >= 0."""
        rows = {}
        for i in range(self.T):
            if i < self.off[0] or i >= self.off[-1] or self.sorted_tok[i] < 0:
                continue
            rows.setdefault(int(np.searchsorted(self.off, i, side="right") - 1), []).append(i)
        return rows

    def oracle_gu_acc(self, xr):
        """gate_up's f32 accumulations (before the output rotation) for every live row: [T, max N], zeros elsewhere."""
        N = max(g.rows for g in self.gu)
        out = np.zeros((self.T, N), np.float32)
        for e, rows in self.live_rows().items():
            g = self.gu[e]
            what = oracle.what_rows(g.codes, g.rows, g.cols, self.bits, self.cb)
            W, C = g.rows // 2, g.cols
            x = f16(xr[rows])
            out[rows, :W] = oracle_acc(x[:, :C], what[:W])
            out[rows, W:2 * W] = oracle_acc(x[:, C:2 * C], what[W:])
        return out

    def oracle_dn_acc(self, h, h_rot):
        """down's f32 accumulations on h (rotated first with down's suh when h_rot = 0): [T, max N]."""
        N = max(d.rows for d in self.dn)
        out = np.zeros((self.T, N), np.float32)
        for e, rows in self.live_rows().items():
            d = self.dn[e]
            what = oracle.what_rows(d.codes, d.rows, d.cols, self.dn_bits, self.cb)
            x = f16(h[rows, :d.cols])
            if not h_rot:
                x = np.stack([oracle.prologue(r, d.suh) for r in x])
            out[rows, :d.rows] = oracle_acc(x, what)
        return out

    def oracle_gate_up_down(self):
        assert self.dn_bits == self.bits, "gate_up_down runs one K; a mixed-K layer is gate_up then down"
        return oracle.run_gate_up_down(self.classes("gu"), self.classes("dn"), self.bits, self.cb, self.x,
                                       self.sorted_tok, self.off, self.top_k, x_bf16=self.x_bf16)


def f16(bits):
    return np.asarray(bits, np.uint16).view(np.float16).astype(np.float32)


def bf16(bits):
    return syn.bf16_to_f32(bits)


def rel_l2(got, want):
    """relative L2 (the reference's device criterion, tests/ref/test_exl3ref.py:336-346: <= 4e-3)."""
    g, w = got.astype(np.float64), want.astype(np.float64)
    return float(np.linalg.norm(g - w) / max(np.linalg.norm(w), 1e-30))


def ordered(bits):
    """fp16 / bf16 bit patterns as integers whose difference counts representable values (ulps) between them."""
    b = np.asarray(bits, np.uint16).astype(np.int32)
    return np.where(b & 0x8000, 0x8000 - b, b)


def narrowed_ok(got, want, fmt):
    """An output narrowed to f16 / bf16 agrees with the oracle's: every element within one unit in the last place of
    its format (a summation order that differs in the f32 rounding can move a value across one rounding boundary) or
    within 1e-4 x RMS in absolute terms (values near zero after cancellation, where an ulp is tiny). Returns the
    number of elements outside the bound."""
    g = f16(got) if fmt == "f16" else bf16(got)
    w = f16(want) if fmt == "f16" else bf16(want)
    rms = float(np.sqrt(np.mean(w.astype(np.float64) ** 2)))
    ulp = np.abs(ordered(got) - ordered(want))
    bad = (ulp > 1) & (np.abs(g.astype(np.float64) - w) > 1e-4 * rms)
    return int(np.count_nonzero(bad))


def oracle_acc(xr, what):
    """acc[r, n] = sum over ascending k of xr[r, k] * what[n, k] in f32, one product and one add a step
    (kernels/exl3ref/ref.c:35-42)."""
    acc = np.zeros((xr.shape[0], what.shape[0]), np.float32)
    for k in range(xr.shape[1]):
        acc = (acc + (xr[:, k:k + 1] * what[None, :, k]).astype(np.float32)).astype(np.float32)
    return acc


def rel_err(got, want):
    """max-abs error over RMS of the reference output (the north star's criterion: <= 2e-3)."""
    rms = float(np.sqrt(np.mean(want.astype(np.float64) ** 2)))
    return float(np.max(np.abs(got.astype(np.float64) - want.astype(np.float64)))) / max(rms, 1e-30)


class Guard:
    """A device buffer between two poisoned MARGIN-byte margins: `view` is the interior (256-byte aligned, as the
    allocator aligns the whole); ok() checks that nothing wrote into the margins."""

    def __init__(self, torch, nbytes, fill=None):
        self.torch = torch
        self.n = int(nbytes)
        self.base = torch.full((self.n + 2 * MARGIN,), POISON, dtype=torch.uint8, device="cuda")
        assert self.base.data_ptr() % 256 == 0
        self.view = self.base[MARGIN:MARGIN + self.n]
        if fill is not None:
            self.view.fill_(fill)

    def ok(self):
        t = self.torch
        return bool(t.all(self.base[:MARGIN] == POISON)) and bool(t.all(self.base[MARGIN + self.n:] == POISON))


class Dev:
    """A case uploaded to the device: stacked stored records and scales, routing, activations. Outputs, scratch and
    counter blocks are guarded (Guard); after every launch the margins and the inputs are checked unchanged."""

    def __init__(self, case: Case, share: "Dev | None" = None):
        import torch
        import exl3c4
        self.case = case
        self.torch, self.ex = torch, exl3c4
        dev = "cuda"
        t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)  # noqa: E731
        self._guards = []
        if share is not None:                           # the same experts (Case.rerouted): share their tables
            self.tabs, self._sums = share.tabs, share._sums
        else:
            self.tabs = {}
            for which in ("gu", "dn"):
                bits = case.bits if which == "gu" else case.dn_bits
                cls = []
                for c in case.classes(which):
                    recs = np.stack([exl3c4.relayout(codes, c["rows"], c["cols"], bits) for codes in c["codes"]])
                    d = {"rows": c["rows"], "cols": c["cols"], "codes": t(recs),
                         "suh": t(c["suh"].view(np.uint16)), "svh": t(c["svh"].view(np.uint16))}
                    if which == "gu":
                        d["suh1"] = t(c["suh1"].view(np.uint16))
                        d["dn_suh"] = t(c["dn_suh"].view(np.uint16))
                    cls.append(d)
                self.tabs[which] = cls
            self._sums = self._table_sums()
        self.x = t(case.x.astype(np.uint16).view(np.int16))
        self.sorted_tok = t(case.sorted_tok)
        self.off = t(case.off)
        self._inputs = (self.x.clone(), self.sorted_tok.clone(), self.off.clone())

    def _table_sums(self):
        torch = self.torch
        return [int(torch.sum(v.view(torch.uint8).to(torch.int64))) for w in ("gu", "dn") for d in self.tabs[w]
                for k, v in sorted(d.items()) if k not in ("rows", "cols")]

    def guard(self, nbytes, fill=None):
        g = Guard(self.torch, nbytes, fill)
        self._guards.append(g)
        return g

    def check_guards(self, what=""):
        """Every guarded buffer's margins intact, and the op's inputs (activations, routing, tables) unchanged."""
        torch = self.torch
        torch.cuda.synchronize()
        bad = [i for i, g in enumerate(self._guards) if not g.ok()]
        assert not bad, f"{what}: a launch wrote into the margins of guarded buffer(s) {bad}"
        x, st, off = self._inputs
        assert torch.equal(self.x, x) and torch.equal(self.sorted_tok, st) and torch.equal(self.off, off), \
            f"{what}: a launch changed its input rows or routing"

    def check_tables(self):
        assert self._table_sums() == self._sums, "a launch changed a weight table"

    def cls(self, which, dn_suh=True):
        out = []
        for d in self.tabs[which]:
            out.append(self.ex.make_class(d["rows"], d["cols"], codes=d["codes"], suh=d["suh"], suh1=d.get("suh1"),
                                          svh=d["svh"], dn_suh=d.get("dn_suh") if dn_suh else None))
        return out

    def scratch(self, o, exact=False):
        """Guarded scratch of the band's size (or exactly this launch's, `exact`), its interior poisoned with 0xFF
        (NaN as f32 and f16): a kernel that read scratch it had not written would show."""
        n = self.ex.launch_scratch_bytes(o) if exact else self.ex.scratch_bytes(o)
        assert n >= 0, f"scratch_bytes {self.ex.STATUS.get(n, n)}"
        return self.guard(max(n, 256), fill=0xFF).view

    def _run(self, o, y, *inputs, expect=0):
        """Launches `o` (whose output is `y`); `inputs`: device tensors the op points to that the caller made for it,
        kept alive with it so that last_acc can launch it again."""
        s = self.scratch(o)
        rc = self.ex.launch(o, s)
        assert rc == expect, f"launch status {self.ex.STATUS.get(rc, rc)}"
        self.torch.cuda.synchronize()
        self.last = (o, y, inputs)
        self.status = self.ex.launch_status(o, s) if rc == 0 else None
        assert self.status in (None, 0), f"gate_up_down's single kernel left status {self.status}"
        self.check_guards("launch")

    def last_acc(self, gemm=0):
        """The f32 accumulations of the last launch: the same op again through exl3c4_launch_checked (which also
        leaves the prefill GEMMs' sums in scratch), whose output must be the production launch's, bit for bit."""
        o, y, _ = self.last
        before = y.clone()
        s = self.scratch(o)
        rc = self.ex.launch_checked(o, s)
        assert rc == 0, f"launch_checked status {self.ex.STATUS.get(rc, rc)}"
        self.torch.cuda.synchronize()
        assert self.torch.equal(y, before), "exl3c4_launch_checked wrote another output than exl3c4_launch"
        self.check_guards("launch_checked")
        return self.ex.partial_sums(o, s, gemm)

    def out(self, cols, fill=0x7E7E, rows=None):
        """A guarded int16 output [rows (default T), cols], prefilled with `fill` (a sentinel the op must overwrite
        where it writes)."""
        rows = self.case.T if rows is None else rows
        g = self.guard(rows * cols * 2)
        v = g.view.view(self.torch.int16).view(rows, cols)
        v.fill_(int(np.uint16(fill & 0xFFFF).view(np.int16)))
        return v

    def prep(self, prefill=0xFFFF):
        c = self.case
        C = max(d["cols"] for d in self.tabs["gu"])
        y = self.out(2 * C, fill=prefill)
        o = self.ex.make_op(self.ex.PREP_GU, c.bits, c.cb, self.cls("gu"), self.x, self.sorted_tok, self.off, y,
                            c.n_tok, c.top_k, x_bf16=c.x_bf16, n_expert=c.n_expert)
        self._run(o, y)
        return y.cpu().numpy().view(np.uint16)

    def gate_up(self, h_rot=0, a_rot=0, xr=None):
        c = self.case
        W = max(d["rows"] for d in self.tabs["gu"]) // 2
        y = self.out(W)
        x = xr if a_rot else self.x
        o = self.ex.make_op(self.ex.GATE_UP, c.bits, c.cb, self.cls("gu"), x, self.sorted_tok, self.off, y,
                            c.n_tok, c.top_k, h_rot=h_rot, a_rot=a_rot, x_bf16=c.x_bf16 and not a_rot,
                            n_expert=c.n_expert)
        self._run(o, y, x)
        return y.cpu().numpy().view(np.uint16)

    def down(self, h, h_rot=0):
        c = self.case
        N = max(d["rows"] for d in self.tabs["dn"])
        y = self.out(N)
        hd = self.torch.from_numpy(np.ascontiguousarray(h).view(np.int16)).to("cuda")
        o = self.ex.make_op(self.ex.DOWN, c.dn_bits, c.cb, self.cls("dn"), hd, self.sorted_tok, self.off, y,
                            c.n_tok, c.top_k, h_rot=h_rot, n_expert=c.n_expert)
        self._run(o, y, hd)
        return y.cpu().numpy().view(np.uint16)

    def gd_op(self, y, M=None):
        """gate_up_down's op over this case, writing y."""
        c = self.case
        dn = [self.ex.make_class(d["rows"], d["cols"], codes=d["codes"], svh=d["svh"]) for d in self.tabs["dn"]]
        return self.ex.make_op(self.ex.GU_DN, c.bits, c.cb, self.cls("gu"), self.x, self.sorted_tok, self.off, y,
                               c.n_tok if M is None else M, c.top_k, dn=dn, x_bf16=c.x_bf16, n_expert=c.n_expert,
                               dn_bits=0 if c.dn_bits == c.bits else c.dn_bits)

    def gate_up_down(self):
        """gate_up_down's output; self.status is then None (two kernels) or 0 (one kernel, which went well)."""
        N = max(d["rows"] for d in self.tabs["dn"])
        y = self.out(N)
        self._run(self.gd_op(y), y)
        return y.cpu().numpy().view(np.uint16)
