"""A seeded sweep of small cases around the launch rules' thresholds, each through every op on the device against the
oracle (gpuchecks.check_all: prep_gu bit-exact, the f32 accumulations within 2e-3 x RMS, narrowed outputs within one
ulp, chains within rel-L2 4e-3, the h_rot / a_rot / pair equalities to the bit, zero rows, a replay).

The batch shapes sit on both sides of each rule the host applies from T = n_tok x top_k and n_expert alone: one row
(gate_up_down's two-launch form that builds h in down's staging), two rows (h by gate_up's epilogue kernel), 31 / 32
/ 33 (gate_up_down as one kernel from EXL3C4_GD_FUSE_MIN_T = 32), 63 / 64 / 65 and the prefill rule's other edge
(the prefill path from T >= 64 and 8 T >= 7 n_expert: exl3c4_prefill_min_rows), and a few larger ones. Everything
else -- K, the codebook, one, two or four classes of their own widths, dropped slots, bf16 input, Zipf routing -- is
drawn from the case's seed and
named in its id, so a failure names what to rerun."""
import numpy as np
import pytest

from cases import Case
from gpuchecks import check_all

pytestmark = pytest.mark.gpu

# (n_tok, top_k, n_expert): T = n_tok x top_k; the prefill path takes T >= 64 and 8 T >= 7 n_expert
SHAPES = [
    (1, 1, 1), (1, 2, 3), (2, 1, 5),                  # T = 1, 2, 2
    (31, 1, 4), (4, 8, 9), (11, 3, 16),               # T = 31, 32, 33: gate_up_down's one-kernel rule
    (9, 7, 8), (8, 8, 73), (8, 8, 74), (13, 5, 8),    # T = 63, 64 (prefill: 512 >= 511), 64 (decode: 512 < 518), 65
    (16, 4, 7), (5, 10, 12), (40, 2, 10),             # T = 64 (prefill), 50, 80 (prefill)
    (24, 6, 200), (32, 4, 16),                        # T = 144 (decode, one kernel: 1152 < 1400), 128 (prefill)
    (3, 10, 10), (16, 2, 5), (7, 9, 30), (12, 8, 12),  # T = 30, 32 (one kernel), 63, 96 (prefill)
    (16, 10, 184), (2, 16, 16), (100, 1, 2), (6, 6, 6),  # T = 160 (decode: 1280 < 1288), 32 (every expert), 100, 36
    (20, 5, 114), (64, 2, 8), (17, 4, 78), (1, 8, 8),   # T = 100 (prefill: 800 >= 798), 128, 68 (decode: 544 < 546), 8
]
# (hidden, width) a class: 640 and 1152 hidden give odd counts of 128-blocks (uneven split-K), a width of 640 ten
# down k-steps
GEOMS = [(128, 128), (256, 128), (256, 256), (384, 128), (128, 256), (640, 384), (1152, 128), (256, 640)]


def _draw(i, n_tok, top_k, n_expert):
    rng = np.random.default_rng(9000 + i)
    n_class = int(rng.choice([1, 2, 4] if n_expert >= 4 else [1, 2] if n_expert >= 2 else [1]))
    geoms = [GEOMS[int(j)] for j in rng.choice(len(GEOMS), n_class)]
    return dict(seed=9100 + i, n_tok=n_tok, top_k=top_k, n_expert=n_expert, geoms=geoms,
                bits=int(rng.integers(2, 9)), cb=str(rng.choice(["mul1", "mul1", "mcg", "3inst"])),
                drop=float(rng.choice([0.0, 0.0, 0.1])), x_bf16=bool(rng.random() < 0.25),
                routing="zipf" if rng.random() < 0.3 and top_k < n_expert else "uniform")


CASES = [_draw(i, *s) for i, s in enumerate(SHAPES)]


def _id(c):
    g = "+".join(f"{h}x{w}" for h, w in c["geoms"])
    return (f"T{c['n_tok'] * c['top_k']}-tok{c['n_tok']}-k{c['top_k']}-E{c['n_expert']}-{g}-K{c['bits']}-{c['cb']}"
            f"{'-drop' if c['drop'] else ''}{'-bf16' if c['x_bf16'] else ''}{'-zipf' if c['routing'] == 'zipf' else ''}")


@pytest.fixture(scope="module")
def torch_cuda():
    torch = pytest.importorskip("torch")
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import exl3c4
    exl3c4.lib()          # raises if the library is not built: no fallback exists
    return torch


@pytest.mark.parametrize("c", CASES, ids=[_id(c) for c in CASES])
def test_sweep_every_op_against_the_oracle(torch_cuda, c):
    print(f"sweep case {_id(c)} seed {c['seed']}", flush=True)
    case = Case(**c)
    dev = check_all(case, _id(c))
    dev.check_guards(_id(c))
