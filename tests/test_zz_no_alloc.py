"""exl3c4_launch_noalloc (GPU): the launch in the library's own device scratch gives exl3c4_launch's bits.

Called through the C-ABI, against exl3c4_launch with the caller's (guarded) scratch on the same inputs, bit for bit:
gate_up_down's single decode kernel (whose counters must start at zero: the launch zeroes them itself), the same op
again on a smaller batch right after (the array keeps the last call's contents: nothing may depend on them), gate_up
alone and the prefill path. And an op whose scratch exceeds the array is refused before anything is written.
"""
import numpy as np
import pytest

from cases import Case, Dev

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def torch_cuda():
    torch = pytest.importorskip("torch")
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import exl3c4
    exl3c4.lib()
    return torch


def _both(dev, make):
    """(noalloc output, launch output) of the op `make(y)` builds, each into its own guarded output."""
    import exl3c4 as ex
    outs = []
    for noalloc in (True, False):
        y = make()
        o = y[1]
        if noalloc:
            assert ex.launch_scratch_bytes(o) <= ex.lib().exl3c4_noalloc_scratch_bytes()
            rc = ex.launch_noalloc(o)
        else:
            rc = ex.launch(o, dev.scratch(o))
        assert rc == 0, f"{'noalloc' if noalloc else 'launch'} status {ex.STATUS.get(rc, rc)}"
        dev.torch.cuda.synchronize()
        outs.append(y[0].cpu().numpy())
    dev.check_guards("noalloc")
    return outs


def test_noalloc_gives_the_launch_bits_on_two_calls_in_a_row_the_second_smaller(torch_cuda):
    import exl3c4 as ex
    big = Case(seed=90, n_tok=8, top_k=10, n_expert=128, geoms=[(2048, 512)], bits=4, cb="mul1", drop=0.05)
    assert not ex.is_prefill(big.T, big.n_expert)       # the decode path: gate_up_down's single kernel at 80 rows
    dev = Dev(big)
    for case, label in ((big, "8 tokens"), (big.rerouted(seed=91, n_tok=3, top_k=10), "3 tokens")):
        d = Dev(case, share=dev)
        print(f"noalloc gate_up_down {label} (T={case.T})", flush=True)

        def make():
            y = d.out(2048)
            return y, d.gd_op(y, M=8)
        a, b = _both(d, make)
        assert np.array_equal(a, b)
        assert not np.all(a == 0x7E7E)


def test_noalloc_gate_up_and_the_prefill_path(torch_cuda):
    import exl3c4 as ex
    case = Case(seed=92, n_tok=64, top_k=2, n_expert=8, geoms=[(256, 256), (384, 128)], bits=3, cb="mcg",
                routing="zipf")
    dev = Dev(case)
    print("noalloc prefill-path gate_up_down, then gate_up", flush=True)

    def make_gd():
        y = dev.out(384)
        return y, dev.gd_op(y)
    a, b = _both(dev, make_gd)
    assert np.array_equal(a, b)

    def make_gu():
        y = dev.out(256)
        return y, ex.make_op(ex.GATE_UP, case.bits, case.cb, dev.cls("gu"), dev.x, dev.sorted_tok, dev.off, y,
                             case.n_tok, case.top_k, h_rot=1)
    a, b = _both(dev, make_gu)
    assert np.array_equal(a, b)


def test_noalloc_refuses_an_op_past_its_scratch_and_writes_nothing(torch_cuda):
    import exl3c4 as ex
    case = Case(seed=93, n_tok=8, top_k=10, n_expert=16, geoms=[(2048, 512)], bits=4, cb="mul1")
    dev = Dev(case)
    o2 = dev.gd_op(dev.out(2048, rows=case.T), M=8)
    o2.x_rows = 0                                  # an op the launch refuses is refused the same way
    assert ex.launch_noalloc(o2) == -1
    big = Case(seed=94, n_tok=96, top_k=10, n_expert=16, geoms=[(2048, 512)], bits=4, cb="mul1")
    dbig = Dev(big)
    yb = dbig.out(2048, fill=0x5A5A)
    ob = dbig.gd_op(yb)
    assert ex.launch_scratch_bytes(ob) > ex.lib().exl3c4_noalloc_scratch_bytes()
    assert ex.launch_noalloc(ob) == -20
    dbig.torch.cuda.synchronize()
    assert np.all(yb.cpu().numpy().view(np.uint16) == 0x5A5A)
    dbig.check_guards("noalloc refusal")
