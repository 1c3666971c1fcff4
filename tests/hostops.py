"""hostops.py -- ops on stand-in device tensors for the host-side tests: fake addresses and shapes only. Every test
that uses them stops at a refusal or a size query, decided on the host before any device call."""
import exl3c4


class Fake:
    """A stand-in for a device tensor: a fake address and a shape; the refusals are decided before any device call."""

    def __init__(self, shape, addr=0x10000, elem=2):
        self.shape, self._addr, self._elem = shape, addr, elem

    def data_ptr(self):
        return self._addr

    def stride(self, d):
        s = 1
        for x in self.shape[d + 1:]:
            s *= x
        return s

    def element_size(self):
        return self._elem

    def numel(self):
        n = 1
        for x in self.shape:
            n *= x
        return n


def op(op=exl3c4.GATE_UP, bits=4, cb="mul1", H=256, W=128, E=4, M=2, top_k=2, h_rot=0, a_rot=0, ycols=None,
       xcols=None, rows_T=None):
    """One op of one class: gate_up [2W, H] (prep_gu, gate_up_down alike) or down [H, W]; E experts; M tokens of
    top_k slots (the band), rows_T sorted rows in this launch (default M * top_k)."""
    rows, cols = (2 * W, H) if op in (exl3c4.GATE_UP, exl3c4.PREP_GU, exl3c4.GU_DN) else (H, W)
    rec = Fake((E, rows * cols * bits // 8), elem=1)
    c = exl3c4.make_class(rows, cols, codes=rec, suh=Fake((E, cols)), suh1=Fake((E, cols)), svh=Fake((E, rows)),
                          dn_suh=Fake((E, W)))
    nT = M * top_k if rows_T is None else rows_T
    x = Fake((M if op != exl3c4.DOWN and not a_rot else nT, xcols or (2 * cols if a_rot else cols)))
    yc = ycols or {exl3c4.GATE_UP: W, exl3c4.DOWN: H, exl3c4.PREP_GU: 2 * H, exl3c4.GU_DN: H}[op]
    y = Fake((nT, yc))
    dn = [exl3c4.make_class(H, W, codes=Fake((E, H * W * bits // 8), elem=1), svh=Fake((E, H)))] \
        if op == exl3c4.GU_DN else None
    return exl3c4.make_op(op, bits, cb, [c], x, Fake((nT,), elem=4), Fake((E + 1,), elem=4), y, M, top_k,
                          h_rot=h_rot, a_rot=a_rot, dn=dn)
