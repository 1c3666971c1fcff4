"""Launches through the radiance plugin rows of libexl3c4.so (RadArgs built as an engine would: operands in schema order,
weight tables, params) give the same bits as the C-ABI entry points (exl3c4_launch), for every op, two-class and
four-class, with the tables in both of the engine's forms: stacked buffers, and pointer tables (stride 0: entry j at
((void**)base)[j], what the engine hands over). The gate_up_down rows' instances (init / fini: a counter-block pool)
give the same bits, keep their blocks zero, and report a wait that gave up as RAD_E_DEVICE on the block's next
launch."""
import ctypes as C
import json
import os

import numpy as np
import pytest

import radplug as rp
from cases import Case, Dev

pytestmark = pytest.mark.gpu
HERE = os.path.dirname(os.path.abspath(__file__))
TABLES = json.load(open(os.path.join(HERE, "golden", "exl3_abi_tables.json")))
PLANES = TABLES["planes"]


@pytest.fixture(scope="module")
def torch_cuda():
    torch = pytest.importorskip("torch")
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import exl3c4
    rp.bind(exl3c4.lib())
    return torch


def _t2(t, dtype):
    return rp.tensor(t.data_ptr(), dtype, list(t.shape), list(t.stride()))


class Plug:
    """One case's operands as plugin tensors."""

    def __init__(self, dev: Dev):
        import exl3c4
        self.dev, self.case, self.lib = dev, dev.case, exl3c4.lib()

    def params(self, si, **extra):
        c = self.case
        gu = self.dev.tabs["gu"]
        g = dict(M=c.n_tok, n_expert=c.n_expert, top_k=c.top_k, dtype=f"exl3k{c.bits}", codebook=c.cb)
        if si % 4 == 1:                                       # down: its own [N, K] = [H, W]
            dn = self.dev.tabs["dn"]
            g.update(N=dn[0]["rows"], K=dn[0]["cols"])
            shapes = [(d["rows"], d["cols"]) for d in dn]
        else:
            g.update(N=gu[0]["rows"], K=gu[0]["cols"])
            shapes = [(d["rows"], d["cols"]) for d in gu]
        if si % 4 == 2:
            del g["N"], g["codebook"]
        if c.n_class == 2:
            if si % 4 != 2:
                g["N_odd"] = shapes[1][0]
            g["K_odd"] = shapes[1][1]
        elif c.n_class == 4:
            for q in range(1, 4):
                if si % 4 != 2:
                    g[f"N_{q}"] = shapes[q][0]
                g[f"K_{q}"] = shapes[q][1]
        g.update(extra)
        return rp.Params(**g)

    def _ptr_table(self, t, dtype, ext):
        """The engine's form of a stacked table t [E, ...]: a device array of E entry addresses, stride 0."""
        torch = self.dev.torch
        step = t.stride(0) * t.element_size()
        addrs = torch.tensor([t.data_ptr() + j * step for j in range(t.shape[0])], dtype=torch.int64, device="cuda")
        self._keep.append(addrs)
        shape = [t.shape[0]] + list(ext)
        return rp.tensor(addrs.data_ptr(), dtype, shape, [0] + [int(np.prod(ext[1:])) if len(ext) > 1 else 1] +
                         ([1] if len(ext) > 1 else []))

    def run(self, si, x, y, ydt, ptr=False, inst=None, **extra):
        """Launch row si with input tensor x (torch) and output y (torch int16); returns the status. ptr: every weight
        table as a pointer table; inst: the row instance to hand over (RadArgs.inst)."""
        self._keep = []
        c = self.case
        schema = TABLES["schemas"][si]
        pos = TABLES["positions"][schema["op"]]
        n = pos["n_opd"]
        ts = (rp.Tensor * n)()
        xdt = rp.BF16 if (c.x_bf16 and si % 4 in (0, 2, 3) and not extra.get("a_rot")) else rp.F16
        ts[pos["x"]] = _t2(x, xdt)
        ts[pos["sorted"]] = _t2(self.dev.sorted_tok, rp.I32)
        ts[pos["offset"]] = _t2(self.dev.off, rp.I32)
        ts[pos["y"]] = _t2(y, ydt)
        which = "dn" if si % 4 == 1 else "gu"
        for cl in range(c.n_class):
            d = self.dev.tabs[which][cl]
            src = {"codes": (d["codes"], rp.U8), "suh": (d["suh"], rp.F16), "svh": (d["svh"], rp.F16)}
            if which == "gu":
                src.update(suh1=(d["suh1"], rp.F16), dn_suh=(d["dn_suh"], rp.F16))
                dd = self.dev.tabs["dn"][cl]
                src.update(dn_codes=(dd["codes"], rp.U8), dn_svh=(dd["svh"], rp.F16))
            r, k = d["rows"], d["cols"]
            ext = {"codes": (r, k), "suh": (k,), "suh1": (k,), "svh": (r,), "dn_suh": (r // 2,),
                   "dn_codes": (k, r // 2), "dn_svh": (k,)}
            for p, name in enumerate(PLANES):
                at = pos["plane"][cl][p]
                if at >= 0 and name in src:
                    t, dt = src[name]
                    if ptr:                                   # entries stored records (codes) / f16 vectors
                        ts[at] = self._ptr_table(t, rp.DT_TRELLIS if "codes" in name else dt, ext[name])
                    else:
                        ts[at] = _t2(t, dt)
        params = self.params(si, **extra)
        args = rp.Args(params.arr, params.n, ts, n, None, 0, inst)
        row = self.lib.rad_kernel_at(si).contents
        need = row.scratch(C.byref(args))     # a geometry the op refuses is refused here too (then so is the launch)
        scratch = self.dev.torch.empty(max(need, 256), dtype=self.dev.torch.uint8, device="cuda")
        args.scratch, args.scratch_bytes = scratch.data_ptr(), scratch.numel()
        stream = self.dev.torch.cuda.current_stream().cuda_stream
        rc = row.launch(C.byref(args), stream)
        self.dev.torch.cuda.synchronize()
        return rc


def _every_op(dev, base, ptr=False):
    """Rows base+0..3 (two-class: 0..3, four-class: 4..7) against the C-ABI results; ptr: pointer tables."""
    p = Plug(dev)
    torch, c = dev.torch, dev.case
    W = max(d["rows"] for d in dev.tabs["gu"]) // 2
    H = max(d["cols"] for d in dev.tabs["gu"])
    N = max(d["rows"] for d in dev.tabs["dn"])
    # prep_gu
    want = dev.prep()
    y = dev.out(2 * H, fill=-1)
    assert p.run(base + 2, dev.x, y, rp.F16, ptr=ptr) == 0
    assert np.array_equal(y.cpu().numpy().view(np.uint16), want)
    xr = torch.from_numpy(want.view(np.int16)).cuda()
    # gate_up, every (h_rot, a_rot)
    for h_rot in (0, 1):
        want = dev.gate_up(h_rot=h_rot)
        for a_rot in (0, 1):
            y = dev.out(W)
            assert p.run(base + 0, xr if a_rot else dev.x, y, rp.F16, ptr=ptr, h_rot=h_rot, a_rot=a_rot) == 0
            assert np.array_equal(y.cpu().numpy().view(np.uint16), want), (h_rot, a_rot)
        if h_rot == 0:
            h0 = want
    # down, both h_rot
    for h_rot in (0, 1):
        h = h0 if h_rot == 0 else dev.gate_up(h_rot=1)
        want = dev.down(h, h_rot=h_rot)
        hd = torch.from_numpy(np.ascontiguousarray(h).view(np.int16)).cuda()
        y = dev.out(N)
        assert p.run(base + 1, hd, y, rp.BF16, ptr=ptr, h_rot=h_rot) == 0
        assert np.array_equal(y.cpu().numpy().view(np.uint16), want), h_rot
    # gate_up_down
    want = dev.gate_up_down()
    y = dev.out(H)
    assert p.run(base + 3, dev.x, y, rp.BF16, ptr=ptr) == 0
    assert np.array_equal(y.cpu().numpy().view(np.uint16), want)
    dev.check_guards("plugin rows")


def test_plugin_rows_two_classes(torch_cuda):
    case = Case(seed=31, n_tok=6, top_k=3, n_expert=9, geoms=[(256, 256), (384, 128)], bits=4, cb="mul1", drop=0.1)
    print("plugin rows: two-class", flush=True)
    _every_op(Dev(case), 0)


def test_plugin_rows_one_class_bf16_mcg(torch_cuda):
    case = Case(seed=32, n_tok=4, top_k=2, n_expert=6, geoms=[(256, 128)], bits=3, cb="mcg", x_bf16=True)
    print("plugin rows: one class, bf16 input, mcg", flush=True)
    _every_op(Dev(case), 0)


def test_plugin_rows_four_classes(torch_cuda):
    case = Case(seed=33, n_tok=5, top_k=4, n_expert=11, geoms=[(256, 128), (256, 256), (128, 128), (256, 128)],
                bits=5, cb="3inst")
    print("plugin rows: four-class", flush=True)
    _every_op(Dev(case), 4)


def test_plugin_refusals_write_nothing(torch_cuda):
    """A refused launch returns its code before writing: the output keeps its fill."""
    case = Case(seed=34, n_tok=3, top_k=2, n_expert=4, geoms=[(128, 128)], bits=4, cb="mul1")
    dev = Dev(case)
    p = Plug(dev)
    W = dev.tabs["gu"][0]["rows"] // 2
    y = dev.out(W, fill=0x1234)
    assert p.run(0, dev.x, y, rp.BF16, h_rot=0, a_rot=0) == rp.E_DTYPE        # gate_up writes f16
    y2 = dev.out(W + 128, fill=0x1234)
    assert p.run(0, dev.x, y2, rp.F16, h_rot=0, a_rot=0) == rp.E_SHAPE        # not the op's width
    assert p.run(0, dev.x, y, rp.F16, h_rot=3, a_rot=0) == rp.E_INVAL
    assert p.run(0, dev.x, y, rp.F16, h_rot=0, a_rot=0, dtype="exl3k9") == rp.E_DTYPE
    assert (y.cpu().numpy() == 0x1234).all() and (y2.cpu().numpy() == 0x1234).all()


@pytest.mark.parametrize("name,base", [("two-class", 0), ("four-class", 4)])
def test_plugin_rows_with_pointer_tables(torch_cuda, name, base):
    """The engine's table form: every plane a device array of entry addresses (stride 0)."""
    geoms = {"two-class": [(256, 256), (384, 128)], "four-class": [(256, 128), (256, 256), (128, 128), (256, 128)]}
    case = Case(seed=35 + base, n_tok=8, top_k=6, n_expert=13, geoms=geoms[name], bits=4, cb="mul1", drop=0.1)
    assert case.T >= 32                                # gate_up_down as its single kernel reads the tables too
    print(f"plugin rows: {name}, pointer tables", flush=True)
    _every_op(Dev(case), base, ptr=True)


def _gd_inst(p, si):
    row = p.lib.rad_kernel_at(si).contents
    params = p.params(si)
    inst = C.c_void_p()
    assert row.init(params.arr, params.n, 0, 1, C.byref(inst)) == 0
    assert inst.value, "the gate_up_down row's init made no instance"
    return row, inst


def test_gate_up_down_row_instance_counter_pool(torch_cuda):
    """The row instance's counter blocks: the same bits as exl3c4_launch, one block per (stream, output), each left
    zero; a launch whose block's flag says a wait gave up returns RAD_E_DEVICE, writes nothing, and the block serves
    the next launch normally."""
    import exl3c4
    case = Case(seed=39, n_tok=8, top_k=10, n_expert=112, geoms=[(512, 256)], bits=4, cb="mul1", drop=0.05)
    assert case.T >= 32 and not exl3c4.is_prefill(case.T, case.n_expert)   # the single kernel: its counter blocks
    dev = Dev(case)
    p = Plug(dev)
    want = dev.gate_up_down()
    row, inst = _gd_inst(p, 3)
    try:
        H = dev.tabs["gu"][0]["cols"]
        y1, y2 = dev.out(H), dev.out(H)
        print("instance: two outputs, two launches each", flush=True)
        for _ in range(2):
            for y in (y1, y2):
                assert p.run(3, dev.x, y, rp.BF16, inst=inst) == 0
                assert np.array_equal(y.cpu().numpy().view(np.uint16), want)
        assert p.lib.exl3c4_plugin_inst_blocks_used(inst) == 2
        assert p.lib.exl3c4_plugin_inst_flag(inst, 0, -1) == 0 and p.lib.exl3c4_plugin_inst_flag(inst, 1, -1) == 0
        print("instance: block 0 flagged as a wait that gave up", flush=True)
        assert p.lib.exl3c4_plugin_inst_flag(inst, 0, 1) == 0       # force the failure path from the host
        y1.fill_(0x1111)
        assert p.run(3, dev.x, y1, rp.BF16, inst=inst) == -21       # RAD_E_DEVICE, nothing written
        assert (y1.cpu().numpy() == 0x1111).all()
        assert p.lib.exl3c4_plugin_inst_flag(inst, 0, -1) == 0
        assert p.run(3, dev.x, y1, rp.BF16, inst=inst) == 0
        assert np.array_equal(y1.cpu().numpy().view(np.uint16), want)
        dev.check_guards("instance launches")
    finally:
        row.fini(inst)


def test_gate_up_down_row_instance_kernel_reports_a_wait_that_gave_up(torch_cuda):
    """The kernel's own failure report, driven from the host without any wait that must time out: before a launch on
    a row instance's block, the host sets the block's status word and drives one live row's counter far negative (no
    count can complete it). The single kernel's waits then give up at their first check (a status word already set
    poisons the block), every kernel exits, and the kernel itself sets the status word and the instance's pinned
    flag (kernels/exl3r4d/exl3r4d.hip:1878-1880 raises the reference's). The block's next launch returns RAD_E_DEVICE
    and writes nothing; the one after it gives the good bits."""
    import exl3c4
    case = Case(seed=41, n_tok=8, top_k=10, n_expert=112, geoms=[(512, 256)], bits=4, cb="mul1", drop=0.05)
    assert case.T >= exl3c4.GD_FUSE_MIN_T and not exl3c4.is_prefill(case.T, case.n_expert)
    dev = Dev(case)
    p = Plug(dev)
    want = dev.gate_up_down()
    hip = exl3c4.hip()
    hip.hipMemcpy.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int]
    hip.hipMemcpy.restype = C.c_int
    row, inst = _gd_inst(p, 3)
    try:
        H = dev.tabs["gu"][0]["cols"]
        y = dev.out(H)
        assert p.run(3, dev.x, y, rp.BF16, inst=inst) == 0        # block 0: (this stream, y)
        assert np.array_equal(y.cpu().numpy().view(np.uint16), want)
        nbytes = C.c_int64()
        blk = p.lib.exl3c4_plugin_inst_block(inst, 0, C.byref(nbytes))
        assert blk and nbytes.value > 0

        def read_block():
            h = np.zeros(nbytes.value // 4, np.int32)
            assert hip.hipMemcpy(h.ctypes.data, blk, nbytes.value, 2) == 0    # device to host
            return h

        def write_word(index, value):
            v = np.array([value], np.int32)
            assert hip.hipMemcpy(blk + 4 * index, v.ctypes.data, 4, 1) == 0   # host to device

        assert not read_block().any()                                # the good launch left its block zero
        live = [i for i in range(case.T) if case.off[0] <= i < case.off[-1] and case.sorted_tok[i] >= 0]
        i = live[len(live) // 2]
        print(f"instance: status word set, row {i}'s counter driven negative, then a launch", flush=True)
        write_word(0, 1)
        write_word((i + 1) * 64, -(1 << 30))
        y.fill_(0x2222)
        assert p.run(3, dev.x, y, rp.BF16, inst=inst) == 0            # the launch itself goes out
        assert read_block()[0] & 1                                   # ... its waits gave up: the status word
        assert p.lib.exl3c4_plugin_inst_flag(inst, 0, -1) == 1       # ... and the kernel's write of the pinned flag
        print("instance: the next launch reports it", flush=True)
        y.fill_(0x1111)
        assert p.run(3, dev.x, y, rp.BF16, inst=inst) == -21          # RAD_E_DEVICE, nothing written
        assert (y.cpu().numpy() == 0x1111).all()
        assert p.lib.exl3c4_plugin_inst_flag(inst, 0, -1) == 0
        assert not read_block().any()                                # the report zeroed the block
        assert p.run(3, dev.x, y, rp.BF16, inst=inst) == 0
        assert np.array_equal(y.cpu().numpy().view(np.uint16), want)
        assert not read_block().any()
        dev.check_guards("instance failure report")
    finally:
        row.fini(inst)
