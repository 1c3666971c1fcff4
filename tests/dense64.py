"""dense64.py -- the routed-expert ops as float64 dense products of the pinned dense weights: the independent
reference the oracle's op level (or_launch, or_gate_up_down) is checked against.

Nothing here comes from the oracle's op code. Each weight is W = diag(svh) Hb W_hat Hb diag(suh) as [n][k]
(common/exl3_decode.h:9-45, exllamav3's order), taken from oracle.decode_rows -- pinned by
tests/test_oracle.py against a float64 product of the golden-pinned W_hat and scipy's Hadamard -- or, where an op's
input arrives rotated already, from W_hat (oracle.what_rows, bit-exact with the golden and the reference C) and
scipy's Hadamard directly. The ops then compose in float64 with no rounding at all:

  prep_gu       xr_m = Hb (x * s_m)                  s_0 = suh, s_1 = suh1           (docs/OPS-exl3.md:96-103)
  gate_up       g = W_gate x, u = W_up x (the gate rows take suh, the up rows suh1), h = silu(g) u
                h_rot = 1: Hb (h * dn_suh)                                             (docs/OPS-exl3.md:104-123)
                a_rot = 1: x arrives as xr: g = svh_g * Hb (W_hat_g xr_0), u likewise with xr_1
  down          y = W_dn h; h_rot = 1: h arrives as Hb (h * suh): y = svh * Hb (W_hat hr)   (docs/OPS-exl3.md:124-140)
  gate_up_down  down(h_rot 1) of gate_up(a_rot 0, h_rot 1): y = W_dn' silu(g) u with W_dn's suh = gate_up's dn_suh
                                                                                       (include/exl3_abi.h:751-800)

Experts are dealt to classes as the engine's tables hold them: expert e in class e % n_class at entry e / n_class
(include/exl3_abi.h:847-853) -- the Case keeps one list of experts, so the class rule never enters here. A row the
runs do not hold, or whose sorted_tok is negative, is zero (include/exl3_abi.h:125-134).

`rounded=True` keeps the reference's rounding points (kernels/exl3ref/ref.c:27-32, 187-225) and nothing else: the
input product f16(x * s) and the rotated input f16(Hb ...) are rounded to f16, gate_up's h to f16 before down's
first step, h_rot's f16(h * dn_suh) and its rotation likewise; every sum and product in between stays float64. The
final f16 / bf16 rounding of an op's output is the caller's (the comparison rounds the float64 value once).

`knobs` plant the mistakes a restatement could make, for the negative controls: "swap_suh" (the gate rows scaled
by suh1), "svh_before_had" (svh applied before the output rotation), "dn_own_suh" (gate_up_down's down scaled by
down's own suh instead of gate_up's dn_suh), "no_silu" (h = g u), "no_xr_round" (with rounded=True, the rotated
input left unrounded).
"""
from __future__ import annotations

import numpy as np
from scipy.linalg import hadamard

import oracle

_H = hadamard(128) / np.sqrt(128.0)


def had(v):
    """Hb over the last axis, in 128-blocks (float64)."""
    v = np.asarray(v, np.float64)
    sh = v.shape
    return (v.reshape(sh[:-1] + (sh[-1] // 128, 128)) @ _H).reshape(sh)


def f16(bits):
    return np.asarray(bits, np.uint16).view(np.float16).astype(np.float64)


def bf16(bits):
    return (np.asarray(bits, np.uint16).astype(np.uint32) << 16).view(np.float32).astype(np.float64)


def silu(g):
    return g / (1.0 + np.exp(-g))


def rnd16(v):
    """float64 -> the nearest f16 (round to nearest even), as float64."""
    return np.asarray(v, np.float64).astype(np.float16).astype(np.float64)


def _f64(v):
    return np.asarray(v, np.float16).astype(np.float64) if np.asarray(v).dtype == np.float16 else \
        f16(np.asarray(v).view(np.uint16))


class Dense:
    def __init__(self, case, knobs=(), rounded=False):
        self.c, self.knobs, self.rounded = case, set(knobs), rounded
        self._w = {}

    def _r(self, v):
        return rnd16(v) if self.rounded else v

    def _rot(self, x, s):
        """Hb (x * s) -- with the reference's roundings f16(Hb f16(x * s)) when rounded."""
        if not self.rounded:
            return had(x * s)
        v = had(rnd16(x * s))
        return v if "no_xr_round" in self.knobs else rnd16(v)

    # ---------------------------------------------------------------- the runs
    def live(self):
        """{row: expert} of the rows an op computes (inside a run, sorted_tok >= 0)."""
        c, out = self.c, {}
        for e in range(c.n_expert):
            for i in range(max(int(c.off[e]), 0), min(int(c.off[e + 1]), c.T)):
                if c.sorted_tok[i] >= 0:
                    out[i] = e
        return out

    def x_row(self, i):
        c = self.c
        t = int(c.sorted_tok[i]) // c.top_k
        return bf16(c.x[t]) if c.x_bf16 else f16(c.x[t])

    # ---------------------------------------------------------------- weights
    def w_gu(self, e):
        """gate_up's dense W [2W, H] (gate rows with suh, up rows with suh1)."""
        key = ("gu", e)
        if key not in self._w:
            g = self.c.gu[e]
            suh, suh1 = (g.suh1, g.suh) if "swap_suh" in self.knobs else (g.suh, g.suh1)
            if "svh_before_had" in self.knobs:
                wh = oracle.what_rows(g.codes, g.rows, g.cols, self.c.bits, self.c.cb).astype(np.float64)
                s = np.where(np.arange(g.rows)[:, None] >= g.rows // 2, _f64(suh1)[None], _f64(suh)[None])
                W = had((_f64(g.svh)[:, None] * had(wh) * s).T).T
            else:
                W = oracle.decode_rows(g.codes, g.rows, g.cols, self.c.bits, self.c.cb, suh, g.svh, suh1=suh1)
            self._w[key] = np.asarray(W, np.float64)
        return self._w[key]

    def w_dn(self, e, suh=None):
        """down's dense W [H, W] with the given input scales (default down's own suh)."""
        key = ("dn", e, None if suh is None else suh.tobytes())
        if key not in self._w:
            d = self.c.dn[e]
            self._w[key] = np.asarray(oracle.decode_rows(d.codes, d.rows, d.cols, self.c.bits, self.c.cb,
                                                         d.suh if suh is None else suh, d.svh), np.float64)
        return self._w[key]

    # ---------------------------------------------------------------- the ops
    def prep(self):
        c = self.c
        C = max(g.cols for g in c.gu)
        out = np.full((c.T, 2 * C), np.nan)
        for e in range(c.n_expert):
            for i in range(max(int(c.off[e]), 0), min(int(c.off[e + 1]), c.T)):
                g = c.gu[e]
                if c.sorted_tok[i] < 0:
                    out[i, :2 * g.cols] = 0.0
                    continue
                x = self.x_row(i)[:g.cols]
                out[i, :g.cols] = self._rot(x, _f64(g.suh))
                out[i, g.cols:2 * g.cols] = self._rot(x, _f64(g.suh1))
        return out                                     # NaN: not written by prep_gu

    def _gu_row(self, i, e, xr=None):
        g = self.c.gu[e]
        Wd = g.rows // 2
        if xr is None and self.rounded:                # the rotated input with the reference's roundings
            x = self.x_row(i)[:g.cols]
            suh, suh1 = (g.suh1, g.suh) if "swap_suh" in self.knobs else (g.suh, g.suh1)
            xr = np.zeros((self.c.T, 2 * g.cols))
            xr[i] = np.concatenate([self._rot(x, _f64(suh)), self._rot(x, _f64(suh1))])
        if xr is None:
            gu = self.w_gu(e) @ self.x_row(i)[:g.cols]
        else:                                          # a_rot: the rotated input as given
            wh = oracle.what_rows(g.codes, g.rows, g.cols, self.c.bits, self.c.cb).astype(np.float64)
            v = np.concatenate([wh[:Wd] @ xr[i, :g.cols], wh[Wd:] @ xr[i, g.cols:2 * g.cols]])
            gu = _f64(g.svh) * np.concatenate([had(v[:Wd]), had(v[Wd:])])
        gt, up = gu[:Wd], gu[Wd:]
        return gt * up if "no_silu" in self.knobs else silu(gt) * up

    def gate_up(self, h_rot=0, xr=None):
        c = self.c
        out = np.zeros((c.T, max(g.rows for g in c.gu) // 2))
        xr64 = None if xr is None else f16(xr)
        for i, e in self.live().items():
            h = self._gu_row(i, e, xr64)
            if h_rot:
                h = self._rot(self._r(h), _f64(c.gu[e].dn_suh))
            out[i, :h.size] = h
        return out

    def down(self, h_bits, h_rot=0):
        c = self.c
        h = f16(h_bits)
        out = np.zeros((c.T, max(d.rows for d in c.dn)))
        for i, e in self.live().items():
            d = c.dn[e]
            if h_rot or self.rounded:                  # the rotated input, as given or rotated here
                hr = h[i, :d.cols] if h_rot else self._rot(h[i, :d.cols], _f64(d.suh))
                wh = oracle.what_rows(d.codes, d.rows, d.cols, c.bits, c.cb).astype(np.float64)
                out[i, :d.rows] = _f64(d.svh) * had(wh @ hr)
            else:
                out[i, :d.rows] = self.w_dn(e) @ h[i, :d.cols]
        return out

    def gate_up_down(self):
        c = self.c
        out = np.zeros((c.T, max(d.rows for d in c.dn)))
        for i, e in self.live().items():
            d, g = c.dn[e], c.gu[e]
            suh = d.suh if "dn_own_suh" in self.knobs else g.dn_suh
            if self.rounded:                           # h f16, then down's first step f16(Hb f16(h dn_suh))
                hr = self._rot(rnd16(self._gu_row(i, e)), _f64(suh))
                wh = oracle.what_rows(d.codes, d.rows, d.cols, c.bits, c.cb).astype(np.float64)
                out[i, :d.rows] = _f64(d.svh) * had(wh @ hr)
            else:
                out[i, :d.rows] = self.w_dn(e, suh) @ self._gu_row(i, e)
        return out
