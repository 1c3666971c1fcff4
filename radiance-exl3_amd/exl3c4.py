"""exl3c4.py -- Python binding of libexl3c4.so (include/exl3c4.h) for tests and the benchmark.

The library is C over HIP; this module only marshals pointers. torch is used for device memory and the stream
(plumbing), never for the computation: every op runs in the library's HIP kernels. If libexl3c4.so is missing this
module raises -- there is no fallback of any kind.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libexl3c4.so")

DOWN, GATE_UP, PREP_GU, GU_DN = 0, 1, 2, 3
K_PREP, K_GATE_UP, K_EPI_GU, K_DOWN, K_GATE_UP_DOWN = 0, 1, 2, 3, 4
GD_FUSE_MIN_T = 32                  # gate_up_down runs as one kernel at decode from this many sorted rows
CB = {"3inst": 0, "mcg": 1, "mul1": 2}
F16, BF16 = 0, 1
STATUS = {0: "OK", -1: "RAD_E_SHAPE", -2: "RAD_E_DTYPE", -3: "RAD_E_ALIGN", -4: "RAD_E_STRIDE", -9: "RAD_E_SCHEMA",
          -12: "RAD_E_INVAL", -18: "RAD_E_UNSUPPORTED", -20: "RAD_E_SCRATCH", -21: "RAD_E_DEVICE",
          -5: "RAD_E_FORMAT", -30: "RAD_E_NOTFOUND", -31: "RAD_E_IO"}
E_FORMAT, E_NOTFOUND, E_IO = -5, -30, -31

_lib = None
_p = C.c_void_p
_i64 = C.c_int64
_i32 = C.c_int32


class Class(C.Structure):
    _fields_ = [("rows", _i32), ("cols", _i32),
                ("codes", _p), ("suh", _p), ("suh1", _p), ("svh", _p), ("dn_suh", _p),
                ("codes_stride", _i64), ("suh_stride", _i64), ("suh1_stride", _i64), ("svh_stride", _i64),
                ("dn_suh_stride", _i64)]


class Op(C.Structure):
    _fields_ = [("op", _i32), ("bits", _i32), ("codebook", _i32), ("n_class", _i32), ("h_rot", _i32), ("a_rot", _i32),
                ("M", _i64), ("n_expert", _i64), ("top_k", _i64),
                ("cls", Class * 4), ("dn", Class * 4),
                ("x", _p), ("x_dtype", _i32), ("x_rows", _i64), ("x_cols", _i64), ("x_pitch", _i64),
                ("sorted_tok", _p), ("expert_offset", _p),
                ("y", _p), ("T", _i64), ("y_cols", _i64), ("y_pitch", _i64), ("dn_bits", _i32)]


def lib():
    """The loaded library; raises when it has not been built (no CPU or torch fallback exists)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is not built: run `python -c 'import __graft_entry__ as g; g.build()'`")
        L = C.CDLL(LIB_PATH)
        L.exl3c4_scratch_bytes.restype = _i64
        L.exl3c4_scratch_bytes.argtypes = [C.POINTER(Op)]
        L.exl3c4_launch_scratch_bytes.restype = _i64
        L.exl3c4_launch_scratch_bytes.argtypes = [C.POINTER(Op)]
        L.exl3c4_scratch_bytes_geom.restype = _i64
        L.exl3c4_scratch_bytes_geom.argtypes = [_i32, _i32, C.POINTER(_i32), C.POINTER(_i32), _i64, _i64, _i64]
        L.exl3c4_launch.restype = C.c_int
        L.exl3c4_launch.argtypes = [C.POINTER(Op), _p, _i64, _p]
        L.exl3c4_launch_noalloc.restype = C.c_int
        L.exl3c4_launch_noalloc.argtypes = [C.POINTER(Op), _p]
        L.exl3c4_noalloc_scratch_bytes.restype = _i64
        L.exl3c4_noalloc_scratch_bytes.argtypes = []
        L.exl3c4_launch_checked.restype = C.c_int
        L.exl3c4_launch_checked.argtypes = [C.POINTER(Op), _p, _i64, _p]
        L.exl3c4_dequant.restype = C.c_int
        L.exl3c4_dequant.argtypes = [_p, _i32, _i32, _i32, _i32, _p, _i64, _p]
        L.exl3c4_record_bytes.restype = _i64
        L.exl3c4_record_bytes.argtypes = [_i64, _i64, _i32]
        L.exl3c4_relayout.restype = C.c_int
        L.exl3c4_relayout.argtypes = [_p, _i64, _i64, _i64, _i32, _p]
        L.exl3c4_unrelayout.restype = C.c_int
        L.exl3c4_unrelayout.argtypes = [_p, _i64, _i64, _i32, _p, _i64]
        L.exl3c4_launch_timed.restype = C.c_int
        L.exl3c4_launch_timed.argtypes = [C.POINTER(Op), _p, _i64, _p, _i32, _p, _p]
        L.exl3c4_scratch_partials.restype = C.c_int
        L.exl3c4_scratch_partials.argtypes = [C.POINTER(Op), _i32, C.POINTER(_i64), C.POINTER(_i64), C.POINTER(_i64),
                                              C.POINTER(_i32)]
        L.exl3c4_router_topk.restype = C.c_int
        L.exl3c4_router_topk.argtypes = [_p, _i32, _i64, _i64, _i64, _i32, _i32, _p, _p, _p]
        L.exl3c4_moe_scatter.restype = C.c_int
        L.exl3c4_moe_scatter.argtypes = [_p, _i64, _i32, _i64, _i64, _p, _p, _p, _p, _p]
        L.exl3c4_router_topk_scatter.restype = C.c_int
        L.exl3c4_router_topk_scatter.argtypes = [_p, _i32, _i64, _i64, _i64, _i32, _i32, _p, _p, _p, _p, _p, _p, _p]
        L.exl3c4_moe_gather.restype = C.c_int
        L.exl3c4_moe_gather.argtypes = [_p, _i32, _i64, _p, _p, _i64, _i32, _i64, _p, _i64, _p]
        L.exl3c4_ctr_bytes.restype = _i64
        L.exl3c4_ctr_bytes.argtypes = [C.POINTER(Op)]
        L.exl3c4_launch_ctr.restype = C.c_int
        L.exl3c4_launch_ctr.argtypes = [C.POINTER(Op), _p, _i64, _p, _p, _i64]
        L.exl3c4_launch_gather.restype = C.c_int
        L.exl3c4_launch_gather.argtypes = [C.POINTER(Op), _p, _i64, _p, _p, _i64, _p, _p, _p, _i64]
        L.exl3c4_scratch_status.restype = C.c_int
        L.exl3c4_scratch_status.argtypes = [C.POINTER(Op), C.POINTER(_i64)]
        L.exl3c4_record_to_codes.restype = C.c_int
        L.exl3c4_record_to_codes.argtypes = [_p, _i64, _i64, _i32, _p, _i64]
        L.exl3c4_ckpt_open.restype = C.c_int
        L.exl3c4_ckpt_open.argtypes = [C.c_char_p, C.POINTER(_p)]
        L.exl3c4_ckpt_close.restype = None
        L.exl3c4_ckpt_close.argtypes = [_p]
        L.exl3c4_ckpt_layers.restype = _i64
        L.exl3c4_ckpt_layers.argtypes = [_p]
        L.exl3c4_import_parse_name.restype = C.c_int
        L.exl3c4_import_parse_name.argtypes = [C.c_char_p, C.POINTER(_i32), C.POINTER(_i64), C.POINTER(_i32)]
        L.exl3c4_import_weight.restype = C.c_int
        L.exl3c4_import_weight.argtypes = [_p, C.c_char_p, _i32, _i32, _i64, _i64, _p, _i64, _p, _p, _p]
        L.exl3c4_prefill_min_rows.restype = _i64
        L.exl3c4_prefill_min_rows.argtypes = [_i64]
        L.exl3c4_check_narrow.restype = C.c_int
        L.exl3c4_check_narrow.argtypes = [_p, _p, _p, _i64, _p]
        L.exl3c4_build_target.restype = C.c_char_p
        L.exl3c4_abi_version.restype = C.c_int
        _lib = L
    return _lib


# ------------------------------------------------------------------------------------------ stored form (host)
def relayout(codes: np.ndarray, rows: int, cols: int, bits: int) -> np.ndarray:
    """Canonical uK plane [rows][row_bytes] -> the stored record (uint8 [rows*cols*bits/8])."""
    codes = np.ascontiguousarray(codes, dtype=np.uint8)
    out = np.zeros(rows * cols * bits // 8, np.uint8)
    rc = lib().exl3c4_relayout(codes.ctypes.data, codes.shape[-1], rows, cols, bits, out.ctypes.data)
    if rc:
        raise ValueError(f"exl3c4_relayout: {STATUS.get(rc, rc)}")
    return out


def unrelayout(record: np.ndarray, rows: int, cols: int, bits: int) -> np.ndarray:
    record = np.ascontiguousarray(record, dtype=np.uint8)
    rb = (cols * bits + 7) // 8
    out = np.zeros((rows, rb), np.uint8)
    rc = lib().exl3c4_unrelayout(record.ctypes.data, rows, cols, bits, out.ctypes.data, rb)
    if rc:
        raise ValueError(f"exl3c4_unrelayout: {STATUS.get(rc, rc)}")
    return out


def record_to_codes(record: np.ndarray, rows: int, cols: int, bits: int) -> np.ndarray:
    """exllamav3's tile record (int16 [cols/16][rows/16][16 K]) -> canonical plane [rows][row_bytes]."""
    record = np.ascontiguousarray(record).view(np.uint16)
    rb = (cols * bits + 7) // 8
    out = np.zeros((rows, rb), np.uint8)
    rc = lib().exl3c4_record_to_codes(record.ctypes.data, rows, cols, bits, out.ctypes.data, rb)
    if rc:
        raise ValueError(f"exl3c4_record_to_codes: {STATUS.get(rc, rc)}")
    return out


# ------------------------------------------------------------------------------------------ the import (host)
class Checkpoint:
    """An EXL3 checkpoint directory opened for import (exl3c4_ckpt_open)."""

    def __init__(self, directory: str):
        self._h = None
        h = _p()
        rc = lib().exl3c4_ckpt_open(os.fsencode(directory), C.byref(h))
        if rc:
            raise OSError(rc, f"exl3c4_ckpt_open: {STATUS.get(rc, rc)}", directory)
        self._h = h

    @property
    def layers(self) -> int:
        return int(lib().exl3c4_ckpt_layers(self._h))

    def close(self):
        if self._h:
            lib().exl3c4_ckpt_close(self._h)
            self._h = None

    def __del__(self):
        self.close()

    def import_weight_rc(self, name: str, bits: int, cb, rows: int, cols: int, planes: dict) -> int:
        """exl3c4_import_weight into the caller's planes (numpy: codes uint8 [rows][row_bytes], suh / suh1 uint16 [cols],
        svh uint16 [rows]; suh1 None for a down weight): the status."""
        cb = CB[cb] if isinstance(cb, str) else cb
        codes = planes["codes"]
        s1 = planes.get("suh1")
        return lib().exl3c4_import_weight(self._h, name.encode(), bits, cb, rows, cols, codes.ctypes.data,
                                         codes.shape[1], planes["suh"].ctypes.data,
                                         None if s1 is None else s1.ctypes.data, planes["svh"].ctypes.data)

    def import_weight(self, name: str, bits: int, cb, rows: int, cols: int) -> dict:
        """The named routed-expert weight as canonical planes (a status other than OK raises)."""
        stacked = ".ffn_gate_up_exps." in name
        planes = {"codes": np.zeros((rows, (cols * bits + 7) // 8), np.uint8), "suh": np.zeros(cols, np.uint16),
                  "suh1": np.zeros(cols, np.uint16) if stacked else None, "svh": np.zeros(rows, np.uint16)}
        rc = self.import_weight_rc(name, bits, cb, rows, cols, planes)
        if rc:
            raise ValueError(f"exl3c4_import_weight({name}): {STATUS.get(rc, rc)}")
        return planes


def parse_weight_name(name: str):
    """(layer, expert, stacked) of a routed-expert weight name, or None (exl3c4_import_parse_name)."""
    layer, expert, stacked = _i32(), _i64(), _i32()
    rc = lib().exl3c4_import_parse_name(name.encode(), C.byref(layer), C.byref(expert), C.byref(stacked))
    return None if rc else (layer.value, expert.value, bool(stacked.value))


# ------------------------------------------------------------------------------------------ device calls
def _stream(stream):
    import torch
    s = torch.cuda.current_stream() if stream is None else stream
    return C.c_void_p(s.cuda_stream)


def _ptr(t):
    return None if t is None else C.c_void_p(t.data_ptr())


def ptr(t):
    return _ptr(t)


def ctypes_ref(o: Op):
    return C.byref(o)


def stream_handle(stream=None):
    return _stream(stream)


# ------------------------------------------------------------------------------------------ HIP events (timing)
_hip = None


def hip():
    """The HIP runtime libexl3c4.so links, for events the caller owns (hipEventCreate / ElapsedTime)."""
    global _hip
    if _hip is None:
        lib()
        _hip = C.CDLL("libamdhip64.so")
        _hip.hipEventCreate.argtypes = [C.POINTER(_p)]
        _hip.hipEventElapsedTime.argtypes = [C.POINTER(C.c_float), _p, _p]
        _hip.hipEventDestroy.argtypes = [_p]
    return _hip


class Event:
    """A raw hipEvent_t (created at once, so a dispatch can stamp it)."""

    def __init__(self):
        self.h = _p()
        if hip().hipEventCreate(C.byref(self.h)):
            raise RuntimeError("hipEventCreate failed")

    def __del__(self):
        if _hip is not None and self.h:
            _hip.hipEventDestroy(self.h)


def elapsed_ms(a: Event, b: Event) -> float:
    ms = C.c_float()
    if hip().hipEventElapsedTime(C.byref(ms), a.h, b.h):
        raise RuntimeError("hipEventElapsedTime failed")
    return float(ms.value)


def launch_timed(o: Op, scratch, kernel: int, ev_start: Event, ev_stop: Event, stream=None) -> int:
    """exl3c4_launch with kernel `kernel` stamping ev_start / ev_stop at its own start and end."""
    n = 0 if scratch is None else scratch.numel()
    return int(lib().exl3c4_launch_timed(C.byref(o), _ptr(scratch), n, _stream(stream), kernel, ev_start.h,
                                         ev_stop.h))


def dequant(record, rows: int, cols: int, bits: int, cb, stream=None):
    """W_hat fp16 bits (torch.int16 [rows, cols]) of a stored record on the device."""
    import torch
    out = torch.empty((rows, cols), dtype=torch.int16, device=record.device)
    rc = lib().exl3c4_dequant(_ptr(record), rows, cols, bits, CB.get(cb, cb), _ptr(out), cols, _stream(stream))
    if rc:
        raise RuntimeError(f"exl3c4_dequant: {STATUS.get(rc, rc)}")
    return out


def prefill_min_rows(n_expert: int) -> int:
    """The least sorted-row count at which an op over n_expert experts takes the prefill path (exl3c4_prefill_min_rows)."""
    return int(lib().exl3c4_prefill_min_rows(n_expert))


def is_prefill(T: int, n_expert: int) -> bool:
    return T >= prefill_min_rows(n_expert)


def check_narrow(values, stream=None):
    """The device's own f32 -> bf16 and f32 -> f16 narrowing (the kernels' outputs' conversions) of a float32 device
    tensor: two uint16 numpy arrays (bf16 bits, f16 bits). A checker's entry (exl3c4_check_narrow)."""
    import torch
    n = values.numel()
    ob = torch.empty(n, dtype=torch.int16, device=values.device)
    oh = torch.empty(n, dtype=torch.int16, device=values.device)
    rc = lib().exl3c4_check_narrow(_ptr(values), _ptr(ob), _ptr(oh), n, _stream(stream))
    if rc:
        raise RuntimeError(f"exl3c4_check_narrow: {STATUS.get(rc, rc)}")
    torch.cuda.synchronize()
    return ob.cpu().numpy().view(np.uint16), oh.cpu().numpy().view(np.uint16)


def make_class(rows, cols, codes=None, suh=None, suh1=None, svh=None, dn_suh=None) -> Class:
    """One class's tables from STACKED device tensors ([entries, ...], contiguous entries)."""
    c = Class()
    c.rows, c.cols = rows, cols
    for name, t in (("codes", codes), ("suh", suh), ("suh1", suh1), ("svh", svh), ("dn_suh", dn_suh)):
        if t is None:
            setattr(c, name, None)
            setattr(c, name + "_stride", 0)
        else:
            setattr(c, name, t.data_ptr())
            setattr(c, name + "_stride", t.stride(0) * t.element_size())
    return c


def make_op(op, bits, cb, classes, x, sorted_tok, expert_offset, y, M, top_k, h_rot=0, a_rot=0, dn=None,
            x_bf16=False, n_expert=None, dn_bits=0) -> Op:
    o = Op()
    o.op, o.bits, o.codebook, o.dn_bits = op, bits, CB.get(cb, cb), dn_bits
    o.n_class, o.h_rot, o.a_rot = len(classes), h_rot, a_rot
    o.M, o.top_k = M, top_k
    o.n_expert = expert_offset.numel() - 1 if n_expert is None else n_expert
    for i, c in enumerate(classes):
        o.cls[i] = c
    for i, c in enumerate(dn or []):
        o.dn[i] = c
    o.x = x.data_ptr()
    o.x_dtype = BF16 if x_bf16 else F16
    o.x_rows, o.x_cols, o.x_pitch = x.shape[0], x.shape[1], x.stride(0)
    o.sorted_tok, o.expert_offset = sorted_tok.data_ptr(), expert_offset.data_ptr()
    o.y = y.data_ptr()
    o.T, o.y_cols, o.y_pitch = y.shape[0], y.shape[1], y.stride(0)
    return o


def scratch_bytes(o: Op) -> int:
    return int(lib().exl3c4_scratch_bytes(C.byref(o)))


def launch_scratch_bytes(o: Op) -> int:
    """The scratch this launch (its T rows) needs; exl3c4_launch refuses below it."""
    return int(lib().exl3c4_launch_scratch_bytes(C.byref(o)))


def launch(o: Op, scratch=None, stream=None) -> int:
    """Runs one op; returns the status (0 OK). `scratch`: a uint8 device tensor of >= scratch_bytes(o)."""
    n = 0 if scratch is None else scratch.numel()
    return int(lib().exl3c4_launch(C.byref(o), _ptr(scratch), n, _stream(stream)))


def launch_noalloc(o: Op, stream=None) -> int:
    """exl3c4_launch_noalloc: the launch in the library's own device scratch (no scratch argument, no allocation)."""
    return int(lib().exl3c4_launch_noalloc(C.byref(o), _stream(stream)))


def launch_checked(o: Op, scratch=None, stream=None) -> int:
    """launch, and a prefill-path launch also leaves its GEMMs' f32 sums in `scratch` for partial_sums."""
    n = 0 if scratch is None else scratch.numel()
    return int(lib().exl3c4_launch_checked(C.byref(o), _ptr(scratch), n, _stream(stream)))


def ctr_bytes(o: Op) -> int:
    """Bytes of the counter block exl3c4_launch_ctr takes for `o` (0: the op keeps no counters)."""
    return int(lib().exl3c4_ctr_bytes(C.byref(o)))


def launch_ctr(o: Op, scratch, ctr, stream=None) -> int:
    """exl3c4_launch_ctr: `ctr` a zeroed uint8 device tensor of >= ctr_bytes(o) bytes, 256-B aligned; left zeroed."""
    n = 0 if scratch is None else scratch.numel()
    m = 0 if ctr is None else ctr.numel()
    return int(lib().exl3c4_launch_ctr(C.byref(o), _ptr(scratch), n, _stream(stream), _ptr(ctr), m))


def launch_gather(o: Op, scratch, ctr, w, row_of, out, stream=None) -> int:
    """exl3c4_launch_gather: launch_ctr, then moe_gather of the op's y (bf16) into out (int16 bits [n_tok, cols], f16)
    with w f32 [n_tok, top_k] and row_of i32; the gather rides in gate_up_down's single kernel when it runs one."""
    n = 0 if scratch is None else scratch.numel()
    m = 0 if ctr is None else ctr.numel()
    return int(lib().exl3c4_launch_gather(C.byref(o), _ptr(scratch), n, _stream(stream), _ptr(ctr), m, _ptr(w),
                                          _ptr(row_of), _ptr(out), out.stride(0)))


def partial_sums(o: Op, scratch, gemm: int = 0):
    """The f32 accumulations a launch left in `scratch` (torch tensor), splits added in the epilogue's order:
    float32 numpy [T, pitch]."""
    off, pitch, ss, n = _i64(), _i64(), _i64(), _i32()
    rc = lib().exl3c4_scratch_partials(C.byref(o), gemm, C.byref(off), C.byref(pitch), C.byref(ss), C.byref(n))
    if rc:
        raise RuntimeError(f"exl3c4_scratch_partials: {STATUS.get(rc, rc)}")
    raw = scratch.cpu().numpy()[off.value:].view(np.float32)
    T = o.T
    acc = raw[: T * pitch.value].reshape(T, pitch.value).copy()
    for s in range(1, n.value):      # columns no launch wrote hold whatever scratch held: no float warnings for them
        with np.errstate(over="ignore", invalid="ignore"):
            acc = (acc + raw[s * ss.value: s * ss.value + T * pitch.value].reshape(T, pitch.value)).astype(np.float32)
    return acc


def launch_status(o: Op, scratch) -> int:
    """The status word gate_up_down's single kernel left in `scratch` (0: good; 1: a wait gave up, the output is
    void), or None when the launch of `o` does not run that kernel."""
    off = _i64()
    if lib().exl3c4_scratch_status(C.byref(o), C.byref(off)):
        return None
    return int(scratch[off.value: off.value + 4].cpu().numpy().view(np.int32)[0])


# ------------------------------------------------------------------------------------------ the routing (device)
F32 = 2


def _dt(t):
    import torch
    return {torch.float32: F32, torch.float16: 0, torch.bfloat16: 1}[t.dtype]


def router_topk(logits, top_k: int, renorm: bool = True, ids=None, w=None, stream=None) -> int:
    """exl3c4_router_topk on a device tensor [n_tok, n_expert] (f32 / f16 / bf16): fills ids (i32) and w (f32)
    [n_tok, top_k]; returns the status."""
    n_tok, n_expert = logits.shape
    return int(lib().exl3c4_router_topk(_ptr(logits), _dt(logits), n_tok, n_expert, logits.stride(0), top_k,
                                        int(renorm), _ptr(ids), _ptr(w), _stream(stream)))


def moe_scatter(ids, n_expert: int, sorted_tok, expert_offset, expert_count=None, row_of=None, expert_base: int = 0,
                stream=None) -> int:
    """exl3c4_moe_scatter on device i32 tensors: ids [n_tok, top_k] in; the rest out."""
    n_tok, top_k = ids.shape
    return int(lib().exl3c4_moe_scatter(_ptr(ids), n_tok, top_k, expert_base, n_expert, _ptr(sorted_tok),
                                        _ptr(expert_offset), _ptr(expert_count), _ptr(row_of), _stream(stream)))


def router_topk_scatter(logits, top_k: int, renorm: bool, ids, w, sorted_tok, expert_offset, expert_count=None,
                        row_of=None, stream=None) -> int:
    """exl3c4_router_topk_scatter: the router and the scatter in one call (one launch up to 16 tokens)."""
    n_tok, n_expert = logits.shape
    return int(lib().exl3c4_router_topk_scatter(_ptr(logits), _dt(logits), n_tok, n_expert, logits.stride(0), top_k,
                                                int(renorm), _ptr(ids), _ptr(w), _ptr(sorted_tok),
                                                _ptr(expert_offset), _ptr(expert_count), _ptr(row_of),
                                                _stream(stream)))


def moe_gather(y, y_bf16: bool, w, row_of, out, stream=None) -> int:
    """exl3c4_moe_gather: y int16 bits [T, cols] (bf16 or f16), w f32 [n_tok, top_k], row_of i32, out int16 bits
    [n_tok, cols] (f16)."""
    n_tok, top_k = w.shape
    return int(lib().exl3c4_moe_gather(_ptr(y), 1 if y_bf16 else 0, y.stride(0), _ptr(w), _ptr(row_of), n_tok, top_k,
                                       y.shape[1], _ptr(out), out.stride(0), _stream(stream)))


def alloc_scratch(o: Op, device="cuda"):
    import torch
    n = scratch_bytes(o)
    if n < 0:
        raise RuntimeError(f"exl3c4_scratch_bytes: {STATUS.get(n, n)}")
    return torch.empty(max(n, 256), dtype=torch.uint8, device=device)
