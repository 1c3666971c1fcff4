"""Launches through the radiance plugin rows of libexl3c4.so (RadArgs built as an engine would: operands in schema order,
stacked weight tables, params) give the same bits as the C-ABI entry points (exl3c4_launch), for every op, two-class
and four-class."""
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

    def run(self, si, x, y, ydt, **extra):
        """Launch row si with input tensor x (torch) and output y (torch int16); returns the status."""
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
            for p, name in enumerate(PLANES):
                at = pos["plane"][cl][p]
                if at >= 0 and name in src:
                    ts[at] = _t2(*src[name])
        params = self.params(si, **extra)
        args = rp.Args(params.arr, params.n, ts, n, None, 0, None)
        row = self.lib.rad_kernel_at(si).contents
        need = row.scratch(C.byref(args))     # a geometry the op refuses is refused here too (then so is the launch)
        scratch = self.dev.torch.empty(max(need, 256), dtype=self.dev.torch.uint8, device="cuda")
        args.scratch, args.scratch_bytes = scratch.data_ptr(), scratch.numel()
        stream = self.dev.torch.cuda.current_stream().cuda_stream
        rc = row.launch(C.byref(args), stream)
        self.dev.torch.cuda.synchronize()
        return rc


def _every_op(dev, base):
    """Rows base+0..3 (two-class: 0..3, four-class: 4..7) against the C-ABI results."""
    p = Plug(dev)
    torch, c = dev.torch, dev.case
    W = max(d["rows"] for d in dev.tabs["gu"]) // 2
    H = max(d["cols"] for d in dev.tabs["gu"])
    N = max(d["rows"] for d in dev.tabs["dn"])
    # prep_gu
    want = dev.prep()
    y = dev.out(2 * H, fill=-1)
    assert p.run(base + 2, dev.x, y, rp.F16) == 0
    assert np.array_equal(y.cpu().numpy().view(np.uint16), want)
    xr = torch.from_numpy(want.view(np.int16)).cuda()
    # gate_up, every (h_rot, a_rot)
    for h_rot in (0, 1):
        want = dev.gate_up(h_rot=h_rot)
        for a_rot in (0, 1):
            y = dev.out(W)
            assert p.run(base + 0, xr if a_rot else dev.x, y, rp.F16, h_rot=h_rot, a_rot=a_rot) == 0
            assert np.array_equal(y.cpu().numpy().view(np.uint16), want), (h_rot, a_rot)
        if h_rot == 0:
            h0 = want
    # down, both h_rot
    for h_rot in (0, 1):
        h = h0 if h_rot == 0 else dev.gate_up(h_rot=1)
        want = dev.down(h, h_rot=h_rot)
        hd = torch.from_numpy(np.ascontiguousarray(h).view(np.int16)).cuda()
        y = dev.out(N)
        assert p.run(base + 1, hd, y, rp.BF16, h_rot=h_rot) == 0
        assert np.array_equal(y.cpu().numpy().view(np.uint16), want), h_rot
    # gate_up_down
    want = dev.gate_up_down()
    y = dev.out(H)
    assert p.run(base + 3, dev.x, y, rp.BF16) == 0
    assert np.array_equal(y.cpu().numpy().view(np.uint16), want)


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
