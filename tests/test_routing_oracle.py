"""The routing around the ops (router, scatter, gather): the oracle's restatements pinned by closed forms, known answers
and library routines (CPU), and the host refusals of the library's entry points (no kernel is launched)."""
import ctypes as C
import math

import numpy as np
import pytest

import oracle


# ------------------------------------------------------------------------------------------ the router
def test_router_uniform_logits_rank_by_id_with_equal_weights():
    """Equal logits tie everywhere: the ids are 0..k-1 (ties to the lower id), p = 1/E, renormalised 1/k."""
    ids, w = oracle.router_topk(np.zeros((3, 16), np.float32), 4, renorm=False)
    assert (ids == np.arange(4)).all()
    assert np.allclose(w, 1 / 16, rtol=0, atol=1e-9)
    ids, w = oracle.router_topk(np.full((2, 16), -3.5, np.float32), 4, renorm=True)
    assert (ids == np.arange(4)).all() and np.allclose(w, 0.25, rtol=0, atol=1e-9)


def test_router_known_answer():
    """logits [0, ln 2, ln 4, 0]: p = [1, 2, 4, 1] / 8; top 2 = ids [2, 1] with p [1/2, 1/4], renormalised [2/3, 1/3]."""
    lg = np.array([[0.0, math.log(2), math.log(4), 0.0]], np.float32)
    ids, w = oracle.router_topk(lg, 2, renorm=False)
    assert ids.tolist() == [[2, 1]]
    assert np.allclose(w, [[0.5, 0.25]], rtol=1e-6)
    ids, w = oracle.router_topk(lg, 2, renorm=True)
    assert np.allclose(w, [[2 / 3, 1 / 3]], rtol=1e-6)
    ids, _ = oracle.router_topk(lg, 4, renorm=True)
    assert ids.tolist() == [[2, 1, 0, 3]]                       # the two tied logits: the lower id first


def test_router_nan_ranks_last():
    ids, _ = oracle.router_topk(np.array([[np.nan, 1.0, 0.0]], np.float32), 3, renorm=False)
    assert ids.tolist() == [[1, 2, 0]]


def test_router_against_scipy_softmax_and_a_sort():
    """Random logits (some quantised so that ties occur): the ids are the first k of a stable sort by descending logit,
    the weights scipy's softmax (float64) at those ids, renormalised."""
    from scipy.special import softmax
    rng = np.random.default_rng(7)
    lg = rng.standard_normal((64, 512)).astype(np.float32)
    lg[::2] = np.round(lg[::2] * 2) / 2                          # ties in half the rows
    for renorm in (False, True):
        ids, w = oracle.router_topk(lg, 10, renorm=renorm)
        want_ids = np.argsort(-lg.astype(np.float64), axis=1, kind="stable")[:, :10]
        assert np.array_equal(ids, want_ids)
        p = softmax(lg.astype(np.float64), axis=1)
        pw = np.take_along_axis(p, want_ids, axis=1)
        if renorm:
            pw = pw / pw.sum(axis=1, keepdims=True)
        assert np.allclose(w, pw, rtol=1e-6, atol=0)


# ------------------------------------------------------------------------------------------ the scatter's extras
def test_scatter_counts_and_row_of_are_the_inverse_permutation():
    rng = np.random.default_rng(8)
    for n_tok, top_k, E, base in ((8, 10, 512, 0), (37, 4, 16, 3), (300, 8, 64, 0)):
        ids = rng.integers(-2, E + base + 2, (n_tok, top_k)).astype(np.int32)
        st, off, cnt, row_of = oracle.moe_scatter_full(ids, E, base)
        st0, off0 = oracle.moe_scatter(ids, E, base)
        assert np.array_equal(st, st0) and np.array_equal(off, off0)
        assert np.array_equal(cnt, np.diff(off))
        flat = ids.reshape(-1) - base
        dropped = (flat < 0) | (flat >= E)
        assert np.all(row_of[dropped] == -1)
        live = np.nonzero(~dropped)[0]
        assert np.array_equal(st[row_of[live]], live)           # row_of inverts sorted_tok
        assert np.array_equal(np.sort(row_of[live]), np.arange(live.size))


# ------------------------------------------------------------------------------------------ the gather
def _bf16_bits(x):
    u = np.asarray(x, np.float32).view(np.uint32)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def test_gather_one_hot_weights_copy_a_row():
    """w = 1 on one slot and 0 elsewhere: out is that slot's row, converted to f16 exactly (values f16 can hold)."""
    rng = np.random.default_rng(9)
    n_tok, top_k, cols = 4, 3, 64
    y = rng.standard_normal((n_tok * top_k, cols)).astype(np.float16)
    row_of = rng.permutation(n_tok * top_k).astype(np.int32)
    w = np.zeros((n_tok, top_k), np.float32)
    w[np.arange(n_tok), np.arange(n_tok) % top_k] = 1.0
    out = oracle.moe_gather(y.view(np.uint16), False, w, row_of, n_tok, top_k)
    for t in range(n_tok):
        assert np.array_equal(out[t], y[row_of[t * top_k + t % top_k]].view(np.uint16))


def test_gather_against_float64_and_dropped_slots():
    rng = np.random.default_rng(10)
    n_tok, top_k, cols = 16, 10, 256
    yf = rng.standard_normal((n_tok * top_k, cols)).astype(np.float32)
    yb = _bf16_bits(yf)
    y64 = (yb.astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    w = rng.random((n_tok, top_k)).astype(np.float32)
    row_of = rng.permutation(n_tok * top_k).astype(np.int32)
    row_of[::7] = -1                                             # dropped pairs add nothing
    out = oracle.moe_gather(yb, True, w, row_of, n_tok, top_k).view(np.float16).astype(np.float64)
    want = np.zeros((n_tok, cols))
    for t in range(n_tok):
        for s in range(top_k):
            r = row_of[t * top_k + s]
            if r >= 0:
                want[t] += float(w[t, s]) * y64[r]
    # f32 accumulation of <= 10 terms, then one f16 rounding: within one f16 ulp of the exact sum
    ulp = np.maximum(np.abs(want), 2.0 ** -14) * 2.0 ** -10
    assert np.all(np.abs(out - want) <= ulp + 1e-6 * np.abs(want))
    # a plausible slip -- the slot order reversed, or a missing -1 test -- is caught by the device tests' bit
    # equality; here the float64 agreement is the anchor


# ------------------------------------------------------------------------------------------ host refusals
class _T:
    def __init__(self, shape, addr=0x10000):
        self.shape, self._addr = shape, addr

    def data_ptr(self):
        return self._addr


def test_routing_refusals_are_decided_on_the_host():
    import exl3c4
    L = exl3c4.lib()
    p = C.c_void_p(0x10000)
    # router: dtype, top_k range, pitch, alignment
    assert L.exl3c4_router_topk(p, 7, 8, 512, 512, 10, 1, p, p, None) == -2
    assert L.exl3c4_router_topk(p, exl3c4.F32, 8, 512, 512, 0, 1, p, p, None) == -1
    assert L.exl3c4_router_topk(p, exl3c4.F32, 8, 512, 512, 65, 1, p, p, None) == -1
    assert L.exl3c4_router_topk(p, exl3c4.F32, 8, 8, 8, 9, 1, p, p, None) == -1
    assert L.exl3c4_router_topk(p, exl3c4.F32, 8, 512, 500, 10, 1, p, p, None) == -4
    assert L.exl3c4_router_topk(C.c_void_p(0x10002), exl3c4.F32, 8, 512, 512, 10, 1, p, p, None) == -3
    assert L.exl3c4_router_topk(p, exl3c4.F32, 8, 512, 512, 10, 2, p, p, None) == -12
    assert L.exl3c4_router_topk(None, exl3c4.F32, 8, 512, 512, 10, 1, p, p, None) == -12
    assert L.exl3c4_router_topk(p, exl3c4.F32, 8, 2048, 2048, 10, 1, p, p, None) == -18   # logits held in registers
    assert L.exl3c4_router_topk_scatter(p, exl3c4.F32, 8, 512, 512, 10, 1, p, p, p, None, None, None, None) == -12
    # scatter: expert count the one-workgroup sort holds
    assert L.exl3c4_moe_scatter(p, 8, 10, 0, 4096, p, p, None, None, None) == -18
    assert L.exl3c4_moe_scatter(p, 8, 0, 0, 512, p, p, None, None, None) == -1
    assert L.exl3c4_moe_scatter(None, 8, 10, 0, 512, p, p, None, None, None) == -12
    # gather: dtype, column multiple, alignment of the 16-byte row loads
    assert L.exl3c4_moe_gather(p, 5, 2048, p, p, 8, 10, 2048, p, 2048, None) == -2
    assert L.exl3c4_moe_gather(p, 1, 2048, p, p, 8, 10, 2044, p, 2048, None) == -1
    assert L.exl3c4_moe_gather(p, 1, 2044, p, p, 8, 10, 2048, p, 2048, None) == -4
    assert L.exl3c4_moe_gather(p, 1, 2052, p, p, 8, 10, 2048, p, 2048, None) == -3
    assert L.exl3c4_moe_gather(C.c_void_p(0x10008), 1, 2048, p, p, 8, 10, 2048, p, 2048, None) == -3
