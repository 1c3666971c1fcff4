"""An imported checkpoint on the device: the fixture's routed experts (tests/golden/exl3_ckpt) through
exl3c4_import_weight -> exl3c4_relayout -> the device decode (exl3c4_dequant), bit-exact against the oracle's decode of
the checkpoint's trellis tensors themselves (common/exl3_decode.c:127-144's exl3_trellis_decode, restated in
oracle/exl3_oracle.c): the whole path from an exllamav3 file to the weights the kernels multiply by."""
import os

import numpy as np
import pytest
from safetensors.numpy import load_file

pytestmark = pytest.mark.gpu
HERE = os.path.dirname(os.path.abspath(__file__))
CKPT = os.path.join(HERE, "golden", "exl3_ckpt")


@pytest.fixture(scope="module")
def torch_cuda():
    torch = pytest.importorskip("torch")
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import exl3c4
    exl3c4.lib()          # raises if the library is not built: no fallback exists
    return torch


@pytest.mark.parametrize("name,prefix,bits,cb", [
    ("blk.0.ffn_gate_up_exps.0.weight", "model.language_model.layers.0.mlp.experts.0", 4, "mul1"),
    ("blk.0.ffn_down_exps.1.weight", "model.language_model.layers.0.mlp.experts.1", 3, "mcg"),
    ("blk.0.ffn_gate_up_exps.2.weight", "model.language_model.layers.0.mlp.experts.2", 2, "3inst"),
    ("blk.2.ffn_down_exps.0.weight", "mtp.layers.0.mlp.experts.0", 4, "mul1"),
])
def test_imported_weights_decode_on_the_device_to_the_trellis_own_w_hat(torch_cuda, name, prefix, bits, cb):
    import exl3c4
    import oracle
    torch = torch_cuda
    print(f"import + dequant {name} K={bits} {cb}", flush=True)
    stacked = "gate_up" in name
    rows, cols = (256, 256) if stacked else (256, 128)
    c = exl3c4.Checkpoint(CKPT)
    planes = c.import_weight(name, bits, cb, rows, cols)
    c.close()
    rec = torch.from_numpy(exl3c4.relayout(planes["codes"], rows, cols, bits)).cuda()
    got = exl3c4.dequant(rec, rows, cols, bits, cb).cpu().numpy().view(np.uint16)
    t = {}
    for f in sorted(os.listdir(CKPT)):
        if f.endswith(".safetensors"):
            t.update(load_file(os.path.join(CKPT, f)))
    parts = ("gate_proj", "up_proj") if stacked else ("down_proj",)
    want = np.concatenate([oracle.trellis_decode(t[f"{prefix}.{p}.trellis"], bits, cb).T for p in parts])
    assert got.shape == want.shape
    assert np.array_equal(got, want), f"{np.count_nonzero(got != want)} of {want.size} differ"
