"""The radiance plugin face of libexl3c4.so (csrc/exl3c4_plugin.c over include/rad_shim.h), on the CPU: identity, the
eight schemas and the operand positions against the reference's own tables (tests/golden/exl3_abi_tables.json, read
from include/exl3_abi.h as text by tests/golden/gen_abi_tables.py), the rows, the shape hook, the parameter parse's
refusals, the scratch hook and the layout hooks. Launches through the rows are in test_gpu_plugin.py."""
import ctypes as C
import json
import os

import numpy as np
import pytest

import radplug as rp

HERE = os.path.dirname(os.path.abspath(__file__))
TABLES = json.load(open(os.path.join(HERE, "golden", "exl3_abi_tables.json")))
PLANES = TABLES["planes"]


@pytest.fixture(scope="module")
def lib():
    import exl3c4
    return rp.bind(exl3c4.lib())


def test_identity(lib):
    assert lib.rad_plugin_abi_version() == rp.RAD_ABI_VERSION
    info = lib.rad_plugin_info().contents
    assert info.build_target == b"gfx950" and info.name == b"exl3c4"
    assert lib.rad_kernel_schema_count() == 8 and lib.rad_kernel_count() == 8
    assert not lib.rad_kernel_schema_at(8) and not lib.rad_kernel_at(-1)


def test_schemas_are_the_references(lib):
    """Op names, parameter specs (key, kind, required), operand lists (name, direction, optional) in order, and the doc
    strings (the engine's loader compares whole schemas)."""
    for i, want in enumerate(TABLES["schemas"]):
        got = rp.schema_of(lib, i)
        assert got == want, f"schema {i} ({want['op']}) differs"


def test_rows(lib):
    for i in range(8):
        row = lib.rad_kernel_at(i).contents
        assert row.op.decode() == TABLES["schemas"][i]["op"]
        assert row.domain == rp.DOMAIN_DEVICE and row.family == b"moe"
        assert row.launch and row.scratch and row.opd_shape and row.layout and row.relayout and row.unrelayout
        assert lib.rad_kernel_concurrent(i) == 1
        keys = {row.constraints[j].key for j in range(row.n_constraints)}
        assert b"dtype" in keys and b"K" in keys
        # the gate_up_down rows keep instance state (a counter-block pool: init allocates, fini frees); no other row
        gd = TABLES["schemas"][i]["op"].startswith("moe_exl3_gate_up_down")
        assert bool(row.init) == gd and bool(row.fini) == gd
        assert b"two launches" not in row.computes


# geometries whose classes all differ, so that each plane table of each class has extents of its own
GEO = {
    "two": dict(M=5, N=512, K=384, N_odd=256, K_odd=256, n_expert=9, top_k=3, dtype="exl3k3", codebook="mcg",
                h_rot=1, a_rot=0),
    "four": dict(M=5, N=512, K=384, N_1=256, K_1=256, N_2=768, K_2=128, N_3=1024, K_3=512, n_expert=11, top_k=3,
                 dtype="exl3k5", codebook="mul1", h_rot=1, a_rot=0),
}


def _class_geom(op, mod4, g):
    if mod4:
        rows = [g["N"], g["N_1"], g["N_2"], g["N_3"]]
        cols = [g["K"], g["K_1"], g["K_2"], g["K_3"]]
    else:
        rows, cols = [g["N"], g["N_odd"]], [g["K"], g["K_odd"]]
    return rows, cols


def _extents(plane, rows, cols):
    return {"codes": (rows, cols), "suh": (1, cols), "suh1": (1, cols), "svh": (rows, 1), "dn_suh": (1, rows // 2),
            "dn_codes": (cols, rows // 2), "dn_svh": (cols, 1)}[plane]


@pytest.mark.parametrize("i", range(8))
def test_positions_via_shape_hook(lib, i):
    """Every position of the reference's Exl3Positions table, asked of this library's shape hook, describes the
    operand that position holds there: the input, the routing, the output, and each class's plane table."""
    op = TABLES["schemas"][i]["op"]
    pos = TABLES["positions"][op]
    mod4 = i >= 4
    g = dict(GEO["four" if mod4 else "two"])
    base = op.replace("moe_exl3_", "").replace("_mod4", "")
    keep = {p[0] for p in TABLES["schemas"][i]["params"]}
    params = rp.Params(**{k: v for k, v in g.items() if k in keep})
    row = lib.rad_kernel_at(i).contents
    rows, cols = _class_geom(base, mod4, g)
    n_cls = 4 if mod4 else 2
    T = g["M"] * g["top_k"]
    xc = max(cols)
    rc, d = rp.shape(row, params, pos["x"])
    assert rc == 0 and d.dtype == rp.F16
    token_rows = base in ("gate_up", "prep_gu", "gate_up_down")
    assert rp.dims(d) == [g["M"] if token_rows else T, xc]
    rc, d = rp.shape(row, params, pos["sorted"])
    assert rc == 0 and d.dtype == rp.I32 and rp.dims(d) == [T]
    rc, d = rp.shape(row, params, pos["offset"])
    assert rc == 0 and rp.dims(d) == [g["n_expert"] + 1] and d.flags & rp.F_IDX_CU
    rc, d = rp.shape(row, params, pos["y"])
    y_cols = {"gate_up": max(rows) // 2, "down": max(rows), "prep_gu": 2 * xc, "gate_up_down": xc}[base]
    assert rc == 0 and rp.dims(d) == [T, y_cols]
    assert d.dtype == (rp.BF16 if base in ("down", "gate_up_down") else rp.F16)
    for c in range(n_cls):
        for p, name in enumerate(PLANES):
            at = pos["plane"][c][p]
            if at < 0:
                continue
            rc, d = rp.shape(row, params, at)
            assert rc == 0, (op, c, name)
            ents = (g["n_expert"] - c + n_cls - 1) // n_cls
            r, cl = _extents(name, rows[c] if base != "prep_gu" else 0, cols[c])
            assert rp.dims(d) == [ents, r, cl], (op, c, name, rp.dims(d))
            bits = int(g["dtype"][-1])
            assert d.dtype == (rp.codes_dtype(bits) if "codes" in name else rp.F16)
    if pos["ids"] >= 0:
        rc, d = rp.shape(row, params, pos["ids"])
        assert rc == 0 and rp.dims(d) == [g["M"], g["top_k"]]
    assert rp.shape(row, params, pos["n_opd"])[0] == rp.E_SHAPE


def test_absent_planes(lib):
    """gate_up's dn_suh tables are absent at h_rot = 0; a two-class op's odd tables without N_odd / K_odd."""
    pos = TABLES["positions"]["moe_exl3_gate_up"]
    row = lib.rad_kernel_at(0).contents
    g = dict(M=4, N=512, K=256, n_expert=6, top_k=2, dtype="exl3k4", codebook="mul1", h_rot=0, a_rot=0)
    params = rp.Params(**g)
    rc, d = rp.shape(row, params, pos["plane"][0][PLANES.index("dn_suh")])
    assert rc == 0 and d.flags & rp.F_ABSENT
    rc, d = rp.shape(row, params, pos["plane"][1][PLANES.index("codes")])
    assert rc == 0 and d.flags & rp.F_ABSENT
    rc, d = rp.shape(row, params, pos["plane"][0][PLANES.index("codes")])
    assert rc == 0 and not d.flags and rp.dims(d) == [6, 512, 256]


def _scratch(row, params, n_t):
    ts = (rp.Tensor * n_t)()
    a = rp.Args(params.arr, params.n, ts, n_t, None, 0, None)
    return row.scratch(C.byref(a))


def test_parse_refusals_through_scratch_hook(lib):
    row = lib.rad_kernel_at(0).contents
    good = dict(M=4, N=512, K=256, n_expert=6, top_k=2, dtype="exl3k4", codebook="mul1", h_rot=0, a_rot=0)
    assert _scratch(row, rp.Params(**good), 14) > 0
    for drop in ("M", "N", "K", "n_expert", "top_k", "dtype", "codebook", "h_rot", "a_rot"):
        bad = {k: v for k, v in good.items() if k != drop}
        assert _scratch(row, rp.Params(**bad), 14) == rp.E_SCHEMA, drop
    assert _scratch(row, rp.Params(**{**good, "dtype": "exl3k9"}), 14) == rp.E_DTYPE
    assert _scratch(row, rp.Params(**{**good, "codebook": "lut"}), 14) == rp.E_DTYPE
    assert _scratch(row, rp.Params(**{**good, "h_rot": 2}), 14) == rp.E_INVAL
    assert _scratch(row, rp.Params(**{**good, "K": 192}), 14) == rp.E_SHAPE
    assert _scratch(row, rp.Params(**{**good, "N": 384}), 14) == rp.E_SHAPE      # gate_up: N % 256
    assert _scratch(row, rp.Params(**{**good, "N_odd": 256}), 14) > 0            # names the odd class
    dn = lib.rad_kernel_at(1).contents
    gd = dict(M=4, N=384, K=256, n_expert=6, top_k=2, dtype="exl3k4", codebook="mul1", h_rot=1)
    assert _scratch(dn, rp.Params(**gd), 10) > 0                                 # down: N % 128
    assert _scratch(dn, rp.Params(**{**gd, "K": 2048}), 10) == rp.E_UNSUPPORTED  # down's k staged whole in LDS


def test_scratch_hook_sizes_from_params(lib):
    """The hook answers exl3c4_scratch_bytes_geom at the band top of M (a range's high bound)."""
    row = lib.rad_kernel_at(3).contents
    g = dict(M=(1, 16), N=1024, K=2048, n_expert=512, top_k=10, dtype="exl3k4", codebook="mul1")
    got = _scratch(row, rp.Params(**g), 18)
    rows = (C.c_int32 * 4)(1024, 1024, 1024, 1024)
    cols = (C.c_int32 * 4)(2048, 2048, 2048, 2048)
    want = lib.exl3c4_scratch_bytes_geom(3, 1, rows, cols, 16, 10, 512)
    assert got == want > 0
    assert lib.exl3c4_scratch_bytes_geom(3, 1, rows, cols, 1, 10, 512) < got


def test_layout_hooks_round_trip(lib):
    """A codes entry is stored as exl3c4_relayout's record; unrelayout gives the canonical plane back; a scale entry is
    its own bytes."""
    import exl3c4
    import exl3c4_synth as syn
    row = lib.rad_kernel_at(1).contents                     # down: codes [N, K]
    pos = TABLES["positions"]["moe_exl3_down"]
    g = dict(M=4, N=256, K=128, n_expert=4, top_k=2, dtype="exl3k3", codebook="mul1", h_rot=0)
    params = rp.Params(**g)
    rng = np.random.default_rng(5)
    plane = syn.random_codes(rng, 256, 128, 3, 1)[0]        # [rows, row_bytes] canonical
    src = rp.tensor(plane.ctypes.data, rp.codes_dtype(3), [256, plane.shape[1]], [plane.shape[1], 1])
    lay = rp.Layout()
    at = pos["plane"][0][PLANES.index("codes")]
    assert row.layout(params.arr, params.n, at, None, None, C.byref(src), 1, C.byref(lay)) == 0
    assert lay.bytes == exl3c4.lib().exl3c4_record_bytes(256, 128, 3) and lay.align == 256
    assert lay.tag == b"exl3c4.trellis.k3" and lay.dtype == rp.DT_TRELLIS
    dst = np.zeros(lay.bytes, np.uint8)
    assert row.relayout(params.arr, params.n, at, None, None, C.byref(src), 1, dst.ctypes.data, dst.size) == 0
    assert np.array_equal(dst, exl3c4.relayout(plane, 256, 128, 3))
    back = np.zeros_like(plane)
    dstt = rp.tensor(back.ctypes.data, rp.codes_dtype(3), [256, back.shape[1]], [back.shape[1], 1])
    assert row.unrelayout(params.arr, params.n, at, None, None, dst.ctypes.data, dst.size, C.byref(dstt), 1) == 0
    assert np.array_equal(back, plane)
    svh = rng.integers(0, 65536, 256, dtype=np.uint16)
    t = rp.tensor(svh.ctypes.data, rp.F16, [256, 1])
    at = pos["plane"][0][PLANES.index("svh")]
    assert row.layout(params.arr, params.n, at, None, None, C.byref(t), 1, C.byref(lay)) == 0
    assert lay.bytes == 512 and lay.tag == b"exl3c4.f16.vec"
    out = np.zeros(256, np.uint16)
    assert row.relayout(params.arr, params.n, at, None, None, C.byref(t), 1, out.ctypes.data, 512) == 0
    assert np.array_equal(out, svh)
    assert row.layout(params.arr, params.n, pos["x"], None, None, C.byref(t), 1, C.byref(lay)) == rp.E_INVAL
