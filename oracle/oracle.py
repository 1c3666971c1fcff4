"""oracle.py -- TEST INFRASTRUCTURE ONLY: numpy-facing ctypes binding of liboracle.so (exl3_oracle.c).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import this module, and only as the checker or
the timed CPU baseline; the product library (radiance-exl3_amd/) never does. Each wrapper names the reference
function it restates (file:line in exl3_oracle.h/.c).
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")
REF_PATH = os.path.join(HERE, "_ref", "libexl3ref_common.so")

CB = {"3inst": 0, "mcg": 1, "mul1": 2}

_lib = None


def build(ref: bool = False) -> None:
    subprocess.run(["make", "-s", "-C", HERE], check=True)
    if ref:
        subprocess.run(["make", "-s", "-C", HERE, "ref"], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        _lib = C.CDLL(LIB_PATH)
        _declare(_lib)
    return _lib


_p = C.c_void_p
_i64 = C.c_int64


def _declare(L):
    L.or_set_threads.argtypes = [C.c_int]
    L.or_get_threads.restype = C.c_int
    L.or_half_to_float.restype = C.c_float
    L.or_half_to_float.argtypes = [C.c_uint16]
    L.or_half_from_double.restype = C.c_uint16
    L.or_half_from_double.argtypes = [C.c_double]
    L.or_f32_to_bf16.restype = C.c_uint16
    L.or_f32_to_bf16.argtypes = [C.c_float]
    L.or_narrow.argtypes = [_p, _p, _p, _i64]
    L.or_codebook_value.restype = C.c_uint16
    L.or_codebook_value.argtypes = [C.c_uint32, C.c_int]
    L.or_codebook_table.argtypes = [C.c_int, _p]
    L.or_pos_to_tile.argtypes = [C.c_int, C.POINTER(C.c_int), C.POINTER(C.c_int)]
    L.or_tile_to_pos.restype = C.c_int
    L.or_tile_to_pos.argtypes = [C.c_int, C.c_int]
    L.or_tile_symbols.argtypes = [_p, C.c_int, _p]
    L.or_tile_pack.argtypes = [_p, C.c_int, _p]
    L.or_tile_states.argtypes = [_p, C.c_int, _p]
    L.or_trellis_decode.restype = C.c_int
    L.or_trellis_decode.argtypes = [_p, _i64, _i64, C.c_int, C.c_int, _p]
    L.or_codes_row_bytes.restype = _i64
    L.or_codes_row_bytes.argtypes = [_i64, C.c_int]
    L.or_codes_get.restype = C.c_uint32
    L.or_codes_get.argtypes = [_p, _i64, C.c_int, _i64, _i64]
    L.or_codes_set.argtypes = [_p, _i64, C.c_int, _i64, _i64, C.c_uint32]
    L.or_record_elems.restype = _i64
    L.or_record_elems.argtypes = [_i64, _i64, C.c_int]
    L.or_codes_to_record.restype = C.c_int
    L.or_codes_to_record.argtypes = [_p, _i64, _i64, _i64, C.c_int, _p]
    L.or_record_to_codes.restype = C.c_int
    L.or_record_to_codes.argtypes = [_p, _i64, _i64, C.c_int, _p, _i64]
    L.or_had128.restype = C.c_int
    L.or_had128.argtypes = [_p, _i64]
    L.or_decode_what_rows.restype = C.c_int
    L.or_decode_what_rows.argtypes = [_p, _i64, _i64, _i64, C.c_int, C.c_int, _i64, _i64, _p]
    L.or_decode_what_rows_f16.restype = C.c_int
    L.or_decode_what_rows_f16.argtypes = [_p, _i64, _i64, _i64, C.c_int, C.c_int, _i64, _i64, _p]
    L.or_decode_rows.restype = C.c_int
    L.or_decode_rows.argtypes = [_p, _i64, _i64, _i64, C.c_int, C.c_int, _p, _p, _p, _i64, _i64, _p]
    L.or_launch.restype = C.c_int
    L.or_launch.argtypes = [_p]
    L.or_gate_up_down.restype = C.c_int
    L.or_gate_up_down.argtypes = [_p, _p]
    L.or_moe_scatter.argtypes = [_p, _i64, _i64, _i64, _i64, _p, _p]
    L.or_moe_scatter_full.argtypes = [_p, _i64, _i64, _i64, _i64, _p, _p, _p, _p]
    L.or_router_topk.argtypes = [_p, _i64, _i64, _i64, C.c_int, C.c_int, _p, _p]
    L.or_moe_gather.argtypes = [_p, C.c_int, _i64, _p, _p, _i64, C.c_int, _i64, _p, _i64]
    L.or_prologue.restype = C.c_int
    L.or_prologue.argtypes = [_p, _p, _i64, _p]


def _ptr(a: np.ndarray):
    assert a.flags["C_CONTIGUOUS"], "oracle arrays must be C-contiguous"
    return a.ctypes.data_as(C.c_void_p)


# ------------------------------------------------------------------------------------------ scalar helpers
def set_threads(n: int) -> None:
    """Threads the op-level oracle spreads live experts over (the outputs do not depend on it)."""
    lib().or_set_threads(int(n))


def get_threads() -> int:
    return int(lib().or_get_threads())


def default_threads() -> int:
    """The host's cores, at most 16 (the GPU box's CPU share)."""
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:
        n = os.cpu_count() or 1
    return max(1, min(16, n))


def half_from_double(x: float) -> int:
    return int(lib().or_half_from_double(float(x)))


def half_to_float(h: int) -> float:
    return float(lib().or_half_to_float(int(h)))


def codebook_value(state: int, cb) -> int:
    return int(lib().or_codebook_value(int(state), CB.get(cb, cb)))


def codebook_table(cb) -> np.ndarray:
    out = np.zeros(65536, np.uint16)
    lib().or_codebook_table(CB.get(cb, cb), _ptr(out))
    return out


def pos_to_tile(p: int):
    r, c = C.c_int(), C.c_int()
    lib().or_pos_to_tile(p, C.byref(r), C.byref(c))
    return r.value, c.value


def tile_to_pos(r: int, c: int) -> int:
    return int(lib().or_tile_to_pos(r, c))


def tile_symbols(tile: np.ndarray, bits: int) -> np.ndarray:
    tile = np.ascontiguousarray(tile, dtype=np.uint16)
    out = np.zeros(256, np.uint8)
    lib().or_tile_symbols(_ptr(tile), bits, _ptr(out))
    return out


def tile_pack(sym: np.ndarray, bits: int) -> np.ndarray:
    sym = np.ascontiguousarray(sym, dtype=np.uint8)
    out = np.zeros(16 * bits, np.uint16)
    lib().or_tile_pack(_ptr(sym), bits, _ptr(out))
    return out


def tile_states(sym: np.ndarray, bits: int) -> np.ndarray:
    sym = np.ascontiguousarray(sym, dtype=np.uint8)
    out = np.zeros(256, np.uint16)
    lib().or_tile_states(_ptr(sym), bits, _ptr(out))
    return out


def trellis_decode(trellis: np.ndarray, bits: int, cb) -> np.ndarray:
    """exllamav3 record int16 [kt][nt][16K] -> W_hat fp16 bits [16kt][16nt] (common/exl3_decode.c:127-144)."""
    t = np.ascontiguousarray(trellis).view(np.uint16)
    kt, nt = t.shape[0], t.shape[1]
    out = np.zeros((16 * kt, 16 * nt), np.uint16)
    rc = lib().or_trellis_decode(_ptr(t), kt, nt, bits, CB.get(cb, cb), _ptr(out))
    if rc:
        raise ValueError(f"or_trellis_decode rc={rc}")
    return out


def row_bytes(cols: int, bits: int) -> int:
    return (cols * bits + 7) // 8


def codes_to_record(codes: np.ndarray, rows: int, cols: int, bits: int) -> np.ndarray:
    codes = np.ascontiguousarray(codes, dtype=np.uint8)
    out = np.zeros(lib().or_record_elems(rows, cols, bits), np.uint16)
    rc = lib().or_codes_to_record(_ptr(codes), codes.shape[-1], rows, cols, bits, _ptr(out))
    if rc:
        raise ValueError(f"or_codes_to_record rc={rc}")
    return out


def record_to_codes(record: np.ndarray, rows: int, cols: int, bits: int) -> np.ndarray:
    record = np.ascontiguousarray(record, dtype=np.uint16)
    out = np.zeros((rows, row_bytes(cols, bits)), np.uint8)
    rc = lib().or_record_to_codes(_ptr(record), rows, cols, bits, _ptr(out), out.shape[1])
    if rc:
        raise ValueError(f"or_record_to_codes rc={rc}")
    return out


def narrow(values: np.ndarray):
    """or_f32_to_bf16 and or_f32_to_f16 of each float32 value (bits passed as they are, nans included): two uint16
    arrays (bf16 bits, f16 bits)."""
    v = np.ascontiguousarray(values, dtype=np.float32)
    bf, h = np.zeros(v.size, np.uint16), np.zeros(v.size, np.uint16)
    lib().or_narrow(_ptr(v), _ptr(bf), _ptr(h), v.size)
    return bf, h


def had128(v: np.ndarray) -> np.ndarray:
    out = np.ascontiguousarray(v, dtype=np.float32).copy()
    rc = lib().or_had128(_ptr(out), out.size)
    if rc:
        raise ValueError("had128 needs a multiple of 128")
    return out


def what_rows(codes: np.ndarray, rows: int, cols: int, bits: int, cb, row0: int = 0, n: int | None = None,
              f16: bool = False) -> np.ndarray:
    """W_hat rows of a canonical plane (common/exl3_decode.c:193-221): f32 values, or fp16 bits with f16=True."""
    codes = np.ascontiguousarray(codes, dtype=np.uint8)
    n = rows - row0 if n is None else n
    if f16:
        out = np.zeros((n, cols), np.uint16)
        rc = lib().or_decode_what_rows_f16(_ptr(codes), codes.shape[-1], rows, cols, bits, CB.get(cb, cb), row0, n,
                                           _ptr(out))
    else:
        out = np.zeros((n, cols), np.float32)
        rc = lib().or_decode_what_rows(_ptr(codes), codes.shape[-1], rows, cols, bits, CB.get(cb, cb), row0, n,
                                       _ptr(out))
    if rc:
        raise ValueError(f"decode_what_rows rc={rc}")
    return out


def decode_rows(codes, rows, cols, bits, cb, suh, svh, suh1=None, row0=0, n=None) -> np.ndarray:
    codes = np.ascontiguousarray(codes, dtype=np.uint8)
    suh = np.ascontiguousarray(suh).view(np.uint16)
    svh = np.ascontiguousarray(svh).view(np.uint16)
    s1 = None if suh1 is None else np.ascontiguousarray(suh1).view(np.uint16)
    n = rows - row0 if n is None else n
    out = np.zeros((n, cols), np.float32)
    rc = lib().or_decode_rows(_ptr(codes), codes.shape[-1], rows, cols, bits, CB.get(cb, cb), _ptr(suh),
                              None if s1 is None else _ptr(s1), _ptr(svh), row0, n, _ptr(out))
    if rc:
        raise ValueError(f"decode_rows rc={rc}")
    return out


def prologue(x: np.ndarray, s: np.ndarray) -> np.ndarray:
    """f16(had128(f16(x * s))) as f32 (kernels/exl3ref/ref.c:27-32); x f32 [n], s f16 [n]."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    s = np.ascontiguousarray(s).view(np.uint16)
    out = np.zeros_like(x)
    if lib().or_prologue(_ptr(x), _ptr(s), x.size, _ptr(out)):
        raise ValueError("prologue needs a multiple of 128")
    return out


def moe_scatter(expert_ids: np.ndarray, n_expert: int, expert_base: int = 0):
    ids = np.ascontiguousarray(expert_ids, dtype=np.int32)
    n_tok, top_k = ids.shape
    st = np.zeros(n_tok * top_k, np.int32)
    off = np.zeros(n_expert + 1, np.int32)
    lib().or_moe_scatter(_ptr(ids), n_tok, top_k, expert_base, n_expert, _ptr(st), _ptr(off))
    return st, off


def moe_scatter_full(expert_ids: np.ndarray, n_expert: int, expert_base: int = 0):
    """or_moe_scatter_full: (sorted_tok, expert_offset, expert_count, row_of)."""
    ids = np.ascontiguousarray(expert_ids, dtype=np.int32)
    n_tok, top_k = ids.shape
    st = np.zeros(n_tok * top_k, np.int32)
    off = np.zeros(n_expert + 1, np.int32)
    cnt = np.zeros(n_expert, np.int32)
    row_of = np.zeros(n_tok * top_k, np.int32)
    lib().or_moe_scatter_full(_ptr(ids), n_tok, top_k, expert_base, n_expert, _ptr(st), _ptr(off), _ptr(cnt),
                              _ptr(row_of))
    return st, off, cnt, row_of


def router_topk(logits: np.ndarray, top_k: int, renorm: bool = True):
    """or_router_topk on f32 logits [n_tok, n_expert]: (ids i32 [n_tok, top_k], w f32 [n_tok, top_k])."""
    lg = np.ascontiguousarray(logits, dtype=np.float32)
    n_tok, n_expert = lg.shape
    ids = np.zeros((n_tok, top_k), np.int32)
    w = np.zeros((n_tok, top_k), np.float32)
    lib().or_router_topk(_ptr(lg), n_tok, n_expert, n_expert, top_k, int(renorm), _ptr(ids), _ptr(w))
    return ids, w


def moe_gather(y_bits: np.ndarray, y_bf16: bool, expert_w: np.ndarray, row_of: np.ndarray, n_tok: int, top_k: int):
    """or_moe_gather: f16 bits [n_tok, cols] from y bits [T, cols] (bf16 or f16)."""
    y = np.ascontiguousarray(y_bits).view(np.uint16)
    w = np.ascontiguousarray(expert_w, dtype=np.float32)
    ro = np.ascontiguousarray(row_of, dtype=np.int32)
    cols = y.shape[1]
    out = np.zeros((n_tok, cols), np.uint16)
    lib().or_moe_gather(_ptr(y), int(y_bf16), cols, _ptr(w), _ptr(ro), n_tok, top_k, cols, _ptr(out), cols)
    return out


# ------------------------------------------------------------------------------------------ the ops
class _Class(C.Structure):
    _fields_ = [("rows", _i64), ("cols", _i64),
                ("codes", _p), ("codes_stride", _i64),
                ("suh", _p), ("suh_stride", _i64),
                ("suh1", _p), ("suh1_stride", _i64),
                ("svh", _p), ("svh_stride", _i64),
                ("dn_suh", _p), ("dn_suh_stride", _i64)]


class _Op(C.Structure):
    _fields_ = [("op", C.c_int), ("bits", C.c_int), ("codebook", C.c_int), ("n_class", C.c_int),
                ("h_rot", C.c_int), ("a_rot", C.c_int), ("n_expert", _i64), ("top_k", _i64),
                ("cls", _Class * 4),
                ("x", _p), ("x_bf16", C.c_int), ("x_rows", _i64), ("x_pitch", _i64),
                ("sorted_tok", _p), ("expert_offset", _p),
                ("y", _p), ("T", _i64), ("y_pitch", _i64)]


OP_DOWN, OP_GATE_UP, OP_PREP_GU = 0, 1, 2


def _fill_class(cs: _Class, cl: dict, keep: list):
    """cl: rows, cols, codes [E][rows][row_bytes] u8, suh [E][cols] f16, suh1, svh [E][rows], dn_suh [E][rows/2]."""
    cs.rows, cs.cols = cl["rows"], cl["cols"]
    for name in ("codes", "suh", "suh1", "svh", "dn_suh"):
        a = cl.get(name)
        if a is None:
            setattr(cs, name, None)
            setattr(cs, name + "_stride", 0)
            continue
        a = np.ascontiguousarray(a)
        if a.dtype == np.float16:
            a = a.view(np.uint16)
        keep.append(a)
        setattr(cs, name, a.ctypes.data)
        setattr(cs, name + "_stride", a[0].nbytes)


def _make_op(op, classes, bits, cb, x, sorted_tok, off, top_k, y, h_rot=0, a_rot=0, x_bf16=False):
    keep = []
    o = _Op()
    o.op, o.bits, o.codebook = op, bits, CB.get(cb, cb)
    o.n_class, o.h_rot, o.a_rot = len(classes), h_rot, a_rot
    o.n_expert, o.top_k = len(off) - 1, top_k
    for c, cl in enumerate(classes):
        _fill_class(o.cls[c], cl, keep)
    xv = np.ascontiguousarray(x).view(np.uint16)
    keep.append(xv)
    o.x, o.x_bf16, o.x_rows, o.x_pitch = xv.ctypes.data, int(x_bf16), xv.shape[0], xv.shape[1]
    st = np.ascontiguousarray(sorted_tok, dtype=np.int32)
    of = np.ascontiguousarray(off, dtype=np.int32)
    keep += [st, of]
    o.sorted_tok, o.expert_offset = st.ctypes.data, of.ctypes.data
    o.y, o.T, o.y_pitch = y.ctypes.data, y.shape[0], y.shape[1]
    return o, keep


def _y_cols(op, classes):
    if op == OP_PREP_GU:
        return 2 * max(c["cols"] for c in classes)
    r = max(c["rows"] for c in classes)
    return r // 2 if op == OP_GATE_UP else r


def run_op(op, classes, bits, cb, x, sorted_tok, off, top_k, T=None, h_rot=0, a_rot=0, x_bf16=False, y=None):
    """prep_gu / gate_up / down as kernels/exl3ref/ref.c computes them. Returns fp16 bits (gate_up h, prep_gu xr) or
    bf16 bits (down y), uint16 [T, y_cols]. `y` (optional) is the prefilled output (prep_gu leaves rows unwritten)."""
    T = len(sorted_tok) if T is None else T
    if y is None:
        y = np.zeros((T, _y_cols(op, classes)), np.uint16)
    o, keep = _make_op(op, classes, bits, cb, x, sorted_tok, off, top_k, y, h_rot, a_rot, x_bf16)
    rc = lib().or_launch(C.byref(o))
    if rc:
        raise RuntimeError(f"or_launch rc={rc}")
    return y


def run_gate_up_down(gu_classes, dn_classes, bits, cb, x, sorted_tok, off, top_k, x_bf16=False):
    T = len(sorted_tok)
    h_dummy = np.zeros((T, _y_cols(OP_GATE_UP, gu_classes)), np.uint16)
    y = np.zeros((T, _y_cols(OP_DOWN, dn_classes)), np.uint16)
    g, k1 = _make_op(OP_GATE_UP, gu_classes, bits, cb, x, sorted_tok, off, top_k, h_dummy, 1, 0, x_bf16)
    d, k2 = _make_op(OP_DOWN, dn_classes, bits, cb, h_dummy, sorted_tok, off, top_k, y, 1, 0, False)
    rc = lib().or_gate_up_down(C.byref(g), C.byref(d))
    if rc:
        raise RuntimeError(f"or_gate_up_down rc={rc}")
    return y
