"""The import of an EXL3 checkpoint's routed experts into canonical planes (exl3c4_import.c), against the reference's
`exl3` quantiser's behaviour (quantizers/exl3/exl3_quant.cpp:12-20, 97-114, 142-296): CPU, nothing is launched.

The fixture (tests/golden/exl3_ckpt, written by tests/golden/gen_exl3_ckpt.py and checked byte for byte against a
fresh run of it here) is a two-shard exllamav3-layout checkpoint: valid experts at K 4 / 3 / 2 with the mul1, mcg and
no (3inst) marker, an MTP-head expert, and one expert per refusal the reference names. Expected planes come from the
fixture's own tensors (read with the safetensors loader) through the oracle's record -> plane walk
(oracle/exl3_oracle.c, pinned against the reference's C and its golden vectors), and the imported plane's W_hat is
checked against the oracle's decode of the trellis itself -- two independent routes to the same weights.
"""
import filecmp
import json
import os

import numpy as np
import pytest
from safetensors.numpy import load_file

import exl3c4
import oracle

HERE = os.path.dirname(os.path.abspath(__file__))
CKPT = os.path.join(HERE, "golden", "exl3_ckpt")
H, W, H1 = 256, 128, 128
TRUNK = "model.language_model.layers.%d.mlp.experts.%d"
MTP = "mtp.layers.0.mlp.experts.%d"


@pytest.fixture(scope="module")
def ckpt():
    c = exl3c4.Checkpoint(CKPT)
    yield c
    c.close()


@pytest.fixture(scope="module")
def tensors():
    out = {}
    for f in sorted(os.listdir(CKPT)):
        if f.endswith(".safetensors"):
            out.update(load_file(os.path.join(CKPT, f)))
    return out


def test_the_fixture_is_what_its_committed_script_writes(tmp_path):
    import importlib.util
    spec = importlib.util.spec_from_file_location("gen_exl3_ckpt", os.path.join(HERE, "golden", "gen_exl3_ckpt.py"))
    gen = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(gen)
    gen.write(str(tmp_path))
    names = sorted(os.listdir(CKPT))
    assert names == sorted(os.listdir(tmp_path))
    for n in names:
        assert filecmp.cmp(os.path.join(CKPT, n), os.path.join(tmp_path, n), shallow=False), n


def test_open_reads_the_layer_count(ckpt):
    assert ckpt.layers == 2


def expected(tensors, prefix, projs, k, bits):
    """Planes from the fixture's tensors: the oracle's record -> plane per projection, the scales as stored."""
    codes, svh = [], []
    for p in projs:
        tr = tensors[f"{prefix}.{p}.trellis"]
        n = tr.shape[1] * 16
        codes.append(oracle.record_to_codes(tr.view(np.uint16), n, k, bits))
        svh.append(tensors[f"{prefix}.{p}.svh"].view(np.uint16))
    return np.concatenate(codes), np.concatenate(svh)


CASES = [  # (weight name, prefix, K, codebook)
    ("blk.0.ffn_gate_up_exps.0.weight", TRUNK % (0, 0), 4, "mul1"),
    ("blk.0.ffn_down_exps.0.weight", TRUNK % (0, 0), 4, "mul1"),
    ("blk.0.ffn_gate_up_exps.1.weight", TRUNK % (0, 1), 3, "mcg"),
    ("blk.0.ffn_down_exps.1.weight", TRUNK % (0, 1), 3, "mcg"),
    ("blk.0.ffn_gate_up_exps.2.weight", TRUNK % (0, 2), 2, "3inst"),
    ("blk.0.ffn_down_exps.2.weight", TRUNK % (0, 2), 2, "3inst"),
    ("blk.2.ffn_gate_up_exps.0.weight", MTP % 0, 4, "mul1"),      # layer index = the layer count: the MTP head
    ("blk.2.ffn_down_exps.0.weight", MTP % 0, 4, "mul1"),
]


@pytest.mark.parametrize("name,prefix,bits,cb", CASES)
def test_import_gives_the_planes_of_the_checkpoints_tensors(ckpt, tensors, name, prefix, bits, cb):
    stacked = "gate_up" in name
    rows, cols = (2 * W, H) if stacked else (H, W)
    planes = ckpt.import_weight(name, bits, cb, rows, cols)
    codes, svh = expected(tensors, prefix, ("gate_proj", "up_proj") if stacked else ("down_proj",), cols, bits)
    assert np.array_equal(planes["codes"], codes)
    assert np.array_equal(planes["svh"], svh)
    first = "gate_proj" if stacked else "down_proj"
    assert np.array_equal(planes["suh"], tensors[f"{prefix}.{first}.suh"].view(np.uint16))
    if stacked:
        assert np.array_equal(planes["suh1"], tensors[f"{prefix}.up_proj.suh"].view(np.uint16))
    # the imported plane decodes to the trellis's own W_hat (the oracle's decode of the record, [k][n])
    parts = ("gate_proj", "up_proj") if stacked else ("down_proj",)
    what = oracle.what_rows(planes["codes"], rows, cols, bits, cb, f16=True)
    ref = np.concatenate([oracle.trellis_decode(tensors[f"{prefix}.{p}.trellis"], bits, cb).T for p in parts])
    assert np.array_equal(what, ref)


def test_the_products_record_walk_agrees_with_the_oracles_both_ways():
    """exl3c4_record_to_codes against the oracle's, and the oracle's plane -> record inverting it (K 1..8)."""
    rng = np.random.default_rng(7)
    for bits in range(1, 9):
        rows, cols = 48, 80
        rec = rng.integers(0, 65536, size=(cols // 16, rows // 16, 16 * bits), dtype=np.uint16)
        got = exl3c4.record_to_codes(rec, rows, cols, bits)
        assert np.array_equal(got, oracle.record_to_codes(rec, rows, cols, bits)), bits
        assert np.array_equal(oracle.codes_to_record(got, rows, cols, bits).reshape(rec.shape), rec), bits


REFUSALS = [  # (weight name, K, codebook, status): one defect each (the fixture's layer 1)
    ("blk.1.ffn_gate_up_exps.0.weight", 2, "mul1", exl3c4.E_FORMAT),       # marker with a wrong value
    ("blk.1.ffn_gate_up_exps.1.weight", 2, "mul1", exl3c4.E_FORMAT),       # both markers
    ("blk.1.ffn_down_exps.2.weight", 2, "mul1", -18),                      # a .bias
    ("blk.1.ffn_down_exps.3.weight", 2, "mul1", -18),                      # half-integer K
    ("blk.1.ffn_gate_up_exps.4.weight", 2, "mul1", exl3c4.E_NOTFOUND),     # up_proj without svh
    ("blk.1.ffn_gate_up_exps.5.weight", 2, "mul1", -1),                    # trellis tiles of another shape
    ("blk.1.ffn_down_exps.6.weight", 2, "mul1", exl3c4.E_FORMAT),          # marker not an I32 scalar
    ("blk.1.ffn_gate_up_exps.7.weight", 2, "mul1", -1),                    # suh of another length
    ("blk.1.ffn_gate_up_exps.8.weight", 2, "mul1", exl3c4.E_FORMAT),       # trellis not I16
    ("blk.1.ffn_gate_up_exps.9.weight", 3, "mul1", -2),                    # K=4 asked as K=3
    ("blk.1.ffn_gate_up_exps.9.weight", 4, "mcg", -2),                     # mul1 asked as mcg
    ("blk.1.ffn_gate_up_exps.10.weight", 2, "mul1", exl3c4.E_NOTFOUND),    # up_proj absent
    ("blk.1.ffn_gate_up_exps.11.weight", 2, "mul1", exl3c4.E_NOTFOUND),    # no such expert
    ("blk.3.ffn_gate_up_exps.0.weight", 2, "mul1", exl3c4.E_NOTFOUND),     # past the layers and the MTP head
]


def poisoned(rows, cols, bits, stacked):
    return {"codes": np.full((rows, (cols * bits + 7) // 8), 0xA5, np.uint8), "suh": np.full(cols, 0xA5A5, np.uint16),
            "suh1": np.full(cols, 0xA5A5, np.uint16) if stacked else None, "svh": np.full(rows, 0xA5A5, np.uint16)}


@pytest.mark.parametrize("name,bits,cb,status", REFUSALS)
def test_each_refusal_of_the_reference_is_kept_and_writes_nothing(ckpt, name, bits, cb, status):
    stacked = "gate_up" in name
    rows, cols = (2 * W, H1) if stacked else (H1, W)
    planes = poisoned(rows, cols, bits, stacked)
    assert ckpt.import_weight_rc(name, bits, cb, rows, cols, planes) == status
    for v in planes.values():
        if v is not None:
            assert np.all(v.view(np.uint8) == 0xA5)


def test_the_control_of_the_refusals_imports():
    """Layer 1's expert 9 is valid at K=4 mul1: the refusals above are its defects, not the fixture's geometry."""
    c = exl3c4.Checkpoint(CKPT)
    p = c.import_weight("blk.1.ffn_gate_up_exps.9.weight", 4, "mul1", 2 * W, H1)
    assert p["codes"].any() and p["svh"].any()


def test_argument_refusals(ckpt):
    p = poisoned(2 * W, H, 4, True)
    assert ckpt.import_weight_rc("blk.0.ffn_gate_up_exps.0.weight", 1, "mul1", 2 * W, H, p) == -12   # K outside 2..8
    assert ckpt.import_weight_rc("blk.0.ffn_gate_up_exps.0.weight", 4, 7, 2 * W, H, p) == -12        # codebook
    assert ckpt.import_weight_rc("blk.0.ffn_gate_up_exps.0.weight", 4, "mul1", 384, H, p) == -1     # halves in 128s
    assert ckpt.import_weight_rc("blk.0.ffn_gate_up_exps.0.weight", 4, "mul1", 2 * W, 200, p) == -1
    assert ckpt.import_weight_rc("blk.0.attn_q.weight", 4, "mul1", 2 * W, H, p) == -18                 # not an expert
    p["suh1"] = None
    assert ckpt.import_weight_rc("blk.0.ffn_gate_up_exps.0.weight", 4, "mul1", 2 * W, H, p) == -12   # no suh1 plane
    assert np.all(p["codes"] == 0xA5)


@pytest.mark.parametrize("name,want", [
    ("blk.0.ffn_gate_up_exps.0.weight", (0, 0, True)),
    ("blk.47.ffn_down_exps.511.weight", (47, 511, False)),
    ("blk.3.ffn_gate_up_exps.12.weight.bias", None),
    ("blk.3.ffn_gate_exps.12.weight", None),
    ("blk.-1.ffn_down_exps.0.weight", None),
    ("blk.0.ffn_down_exps.0.weights", None),
    ("", None),
])
def test_weight_names_parse_as_the_reference_parses_them(name, want):
    assert exl3c4.parse_weight_name(name) == want


def write_ckpt(d, config, tensors=None, index=None):
    os.makedirs(d, exist_ok=True)
    if config is not None:
        with open(os.path.join(d, "config.json"), "w") as f:
            json.dump(config, f)
    if tensors is not None:
        from safetensors.numpy import save_file
        save_file(tensors, os.path.join(d, "model.safetensors"))
    if index is not None:
        with open(os.path.join(d, "model.safetensors.index.json"), "w") as f:
            json.dump(index, f)


EXL3_CFG = {"quantization_config": {"quant_method": "exl3"}, "num_hidden_layers": 1}


def test_open_refuses_what_is_not_an_exl3_checkpoint(tmp_path):
    cases = {
        "no_config": (None, None, None),
        "gptq": ({"quantization_config": {"quant_method": "gptq"}, "num_hidden_layers": 1}, {}, None),
        "no_layers": ({"quantization_config": {"quant_method": "exl3"}}, {}, None),
        "no_tensors": (EXL3_CFG, None, None),
        "bad_index": (EXL3_CFG, None, {"weight_map": ["not", "an", "object"]}),
    }
    for name, (cfg, tens, idx) in cases.items():
        d = str(tmp_path / name)
        write_ckpt(d, cfg, {"x": np.zeros(1, np.float16)} if tens is not None else None, idx)
        with pytest.raises(OSError) as e:
            exl3c4.Checkpoint(d)
        assert e.value.errno == exl3c4.E_FORMAT, name
    bad = tmp_path / "bad_json"
    bad.mkdir()
    (bad / "config.json").write_text('{"quantization_config": {"quant_method": "exl3"}, "num_hidden_layers": 1')
    with pytest.raises(OSError):
        exl3c4.Checkpoint(str(bad))


def test_a_single_file_checkpoint_and_a_truncated_header(tmp_path, tensors):
    """model.safetensors without an index; then the same file cut inside its header (refused at open)."""
    prefix = TRUNK % (0, 0)
    one = {k.replace(prefix, MTP % 3): v for k, v in tensors.items() if k.startswith(prefix + ".")}
    d = str(tmp_path / "single")
    write_ckpt(d, {"quantization_config": {"quant_method": "exl3"}, "text_config": {"num_hidden_layers": 5}}, one)
    c = exl3c4.Checkpoint(d)
    assert c.layers == 5
    p = c.import_weight("blk.5.ffn_down_exps.3.weight", 4, "mul1", H, W)   # the MTP head of a 5-layer model
    codes, svh = expected(tensors, prefix, ("down_proj",), W, 4)
    assert np.array_equal(p["codes"], codes) and np.array_equal(p["svh"], svh)
    c.close()
    path = os.path.join(d, "model.safetensors")
    data = open(path, "rb").read()
    open(path, "wb").write(data[:40])
    with pytest.raises(OSError) as e:
        exl3c4.Checkpoint(d)
    assert e.value.errno == exl3c4.E_FORMAT


def test_an_index_naming_a_missing_shard_fails_at_the_lookup(tmp_path):
    d = str(tmp_path / "missing_shard")
    write_ckpt(d, EXL3_CFG, None, {"weight_map": {f"{MTP % 0}.down_proj.trellis": "model-00009.safetensors"}})
    c = exl3c4.Checkpoint(d)
    p = poisoned(H, W, 4, False)
    assert c.import_weight_rc("blk.1.ffn_down_exps.0.weight", 4, "mul1", H, W, p) == exl3c4.E_FORMAT
