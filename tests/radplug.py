"""ctypes mirror of include/rad_shim.h, for the tests of libexl3c4.so's radiance plugin face (test infrastructure)."""
from __future__ import annotations

import ctypes as C

import numpy as np

RAD_ABI_VERSION = 17
OK, E_SHAPE, E_DTYPE, E_ALIGN, E_STRIDE, E_SCHEMA, E_INVAL, E_UNSUPPORTED, E_SCRATCH = 0, -1, -2, -3, -4, -9, -12, -18, -20
F32, F16, BF16, I32, I64, U8 = 1, 2, 3, 4, 5, 6
U = {k: 10 + k for k in range(1, 8)}                     # RAD_U1..RAD_U7 = 11..17 (RAD_U8 is U8)
DT_PRIVATE = 64
DT_TRELLIS = DT_PRIVATE + 1
P_INT, P_STR = 1, 2
OPD_IN, OPD_OUT, OPD_WTAB = 1, 2, 3
FILL_NORMAL, FILL_INDEX = 1, 2
F_ABSENT, F_IDX_CU = 1, 2
DOMAIN_DEVICE = 2
MAX_RANK = 8


def codes_dtype(bits):
    return U8 if bits == 8 else U[bits]


class Param(C.Structure):
    _fields_ = [("key", C.c_char_p), ("kind", C.c_int), ("ival", C.c_int64), ("ihi", C.c_int64),
                ("sval", C.c_char_p), ("fval", C.c_double)]


class ParamSpec(C.Structure):
    _fields_ = [("key", C.c_char_p), ("kind", C.c_int), ("required", C.c_int), ("role", C.c_int)]


class OperandSpec(C.Structure):
    _fields_ = [("name", C.c_char_p), ("dir", C.c_int), ("optional", C.c_int)]


class OpSchema(C.Structure):
    _fields_ = [("op", C.c_char_p), ("params", C.POINTER(ParamSpec)), ("n_params", C.c_int),
                ("operands", C.POINTER(OperandSpec)), ("n_operands", C.c_int), ("doc", C.c_char_p)]


class Tensor(C.Structure):
    _fields_ = [("data", C.c_void_p), ("dtype", C.c_uint32), ("rank", C.c_uint32),
                ("shape", C.c_int64 * MAX_RANK), ("stride", C.c_int64 * MAX_RANK)]


class Args(C.Structure):
    _fields_ = [("p", C.POINTER(Param)), ("n_p", C.c_int), ("t", C.POINTER(Tensor)), ("n_t", C.c_int),
                ("scratch", C.c_void_p), ("scratch_bytes", C.c_int64), ("inst", C.c_void_p)]


class OpdDesc(C.Structure):
    _fields_ = [("dtype", C.c_uint32), ("rank", C.c_uint32), ("shape", C.c_int64 * MAX_RANK), ("fill", C.c_uint32),
                ("flags", C.c_uint32), ("idx_max", C.c_int64), ("idx_const", C.c_int64)]


class EncPlane(C.Structure):
    _fields_ = [("name", C.c_char * 64), ("dtype", C.c_uint32), ("tile_r", C.c_int), ("tile_c", C.c_int)]


class Encoding(C.Structure):
    _fields_ = [("scheme", C.c_char * 64), ("transform", C.c_char * 64), ("n_planes", C.c_int),
                ("plane", EncPlane * 8)]


class Layout(C.Structure):
    _fields_ = [("tag", C.c_char * 64), ("dtype", C.c_uint32), ("bytes", C.c_int64), ("align", C.c_int64)]


class Constraint(C.Structure):
    _fields_ = [("key", C.c_char_p), ("kind", C.c_int), ("v", C.c_int64), ("set", C.c_char_p)]


INIT = C.CFUNCTYPE(C.c_int, C.POINTER(Param), C.c_int, C.c_int, C.c_int, C.POINTER(C.c_void_p))
FINI = C.CFUNCTYPE(None, C.c_void_p)
LAUNCH = C.CFUNCTYPE(C.c_int, C.POINTER(Args), C.c_void_p)
SCRATCH = C.CFUNCTYPE(C.c_int64, C.POINTER(Args))
SHAPE = C.CFUNCTYPE(C.c_int, C.POINTER(Param), C.c_int, C.c_int, C.POINTER(OpdDesc))
LAYOUT = C.CFUNCTYPE(C.c_int, C.POINTER(Param), C.c_int, C.c_int, C.POINTER(Encoding), C.POINTER(C.c_int),
                     C.POINTER(Tensor), C.c_int, C.POINTER(Layout))
RELAYOUT = C.CFUNCTYPE(C.c_int, C.POINTER(Param), C.c_int, C.c_int, C.POINTER(Encoding), C.POINTER(C.c_int),
                       C.POINTER(Tensor), C.c_int, C.c_void_p, C.c_int64)
UNRELAYOUT = C.CFUNCTYPE(C.c_int, C.POINTER(Param), C.c_int, C.c_int, C.POINTER(Encoding), C.POINTER(C.c_int),
                         C.c_void_p, C.c_int64, C.POINTER(Tensor), C.c_int)


class KernelInfo(C.Structure):
    _fields_ = [("name", C.c_char_p), ("op", C.c_char_p), ("family", C.c_char_p), ("computes", C.c_char_p),
                ("shape", C.c_char_p), ("dtypes", C.c_char_p), ("domain", C.c_int), ("priority", C.c_int),
                ("constraints", C.POINTER(Constraint)), ("n_constraints", C.c_int),
                ("init", INIT), ("fini", FINI), ("launch", LAUNCH), ("scratch", SCRATCH),
                ("layout", LAYOUT), ("relayout", RELAYOUT), ("opd_shape", SHAPE), ("unrelayout", UNRELAYOUT)]


class PluginInfo(C.Structure):
    _fields_ = [("kind", C.c_int), ("name", C.c_char_p), ("version", C.c_char_p), ("desc", C.c_char_p),
                ("build_target", C.c_char_p)]


def bind(lib):
    lib.rad_plugin_abi_version.restype = C.c_uint32
    lib.rad_plugin_info.restype = C.POINTER(PluginInfo)
    lib.rad_kernel_schema_count.restype = C.c_int
    lib.rad_kernel_schema_at.restype = C.POINTER(OpSchema)
    lib.rad_kernel_schema_at.argtypes = [C.c_int]
    lib.rad_kernel_count.restype = C.c_int
    lib.rad_kernel_at.restype = C.POINTER(KernelInfo)
    lib.rad_kernel_at.argtypes = [C.c_int]
    lib.rad_kernel_concurrent.argtypes = [C.c_int]
    lib.exl3c4_plugin_inst_flag.restype = C.c_int32
    lib.exl3c4_plugin_inst_flag.argtypes = [C.c_void_p, C.c_int32, C.c_int32]
    lib.exl3c4_plugin_inst_blocks_used.restype = C.c_int32
    lib.exl3c4_plugin_inst_blocks_used.argtypes = [C.c_void_p]
    lib.exl3c4_plugin_inst_block.restype = C.c_void_p
    lib.exl3c4_plugin_inst_block.argtypes = [C.c_void_p, C.c_int32, C.POINTER(C.c_int64)]
    lib.exl3c4_scratch_bytes_geom.restype = C.c_int64
    lib.exl3c4_scratch_bytes_geom.argtypes = [C.c_int32, C.c_int32, C.POINTER(C.c_int32), C.POINTER(C.c_int32),
                                              C.c_int64, C.c_int64, C.c_int64]
    return lib


class Params:
    """A RadParam array that owns its strings."""

    def __init__(self, **kw):
        self._keep = []
        arr = (Param * max(len(kw), 1))()
        for i, (k, v) in enumerate(kw.items()):
            kb = k.encode()
            self._keep.append(kb)
            if isinstance(v, str):
                vb = v.encode()
                self._keep.append(vb)
                arr[i] = Param(kb, P_STR, 0, 0, vb, 0.0)
            elif isinstance(v, tuple):                       # an int range (lo, hi)
                arr[i] = Param(kb, P_INT, v[0], v[1], None, 0.0)
            else:
                arr[i] = Param(kb, P_INT, int(v), 0, None, 0.0)
        self.arr, self.n = arr, len(kw)


def tensor(data_ptr, dtype, shape, stride=None):
    t = Tensor()
    t.data = data_ptr
    t.dtype = dtype
    t.rank = len(shape)
    if stride is None:
        stride, s = [], 1
        for d in reversed(shape):
            stride.insert(0, s)
            s *= d
    for r, (d, st) in enumerate(zip(shape, stride)):
        t.shape[r] = d
        t.stride[r] = st
    return t


def schema_of(lib, i):
    s = lib.rad_kernel_schema_at(i).contents
    params = [[s.params[j].key.decode(), {P_INT: "INT", P_STR: "STR"}[s.params[j].kind],
               "REQUIRED" if s.params[j].required else "OPTIONAL"] for j in range(s.n_params)]
    opds = [[s.operands[j].name.decode(), {OPD_IN: "IN", OPD_OUT: "OUT", OPD_WTAB: "WTAB"}[s.operands[j].dir],
             int(s.operands[j].optional)] for j in range(s.n_operands)]
    return {"op": s.op.decode(), "params": params, "operands": opds, "doc": s.doc.decode()}


def shape(row, params, operand):
    d = OpdDesc()
    rc = row.opd_shape(params.arr, params.n, operand, C.byref(d))
    return rc, d


def dims(d):
    return [d.shape[r] for r in range(d.rank)]


def as_np(d):
    return np.array(dims(d), dtype=np.int64)
