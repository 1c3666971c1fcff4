#!/usr/bin/env python3
"""gen_exl3_ckpt.py -- writes tests/golden/exl3_ckpt/, a small synthetic EXL3 checkpoint in exllamav3's safetensors
layout (the form turboderp's conversions are published in), for the import tests (tests/test_import.py).

The layout followed (quantizers/exl3/exl3_quant.cpp:1-20, 142-296; quantizers/exl3/exl3_src.h:1-10):
  config.json                      quantization_config.quant_method "exl3"; text_config.num_hidden_layers
  model.safetensors.index.json     weight_map: tensor name -> shard file
  model-0000N-of-00002.safetensors the tensors
  <P>.E.{gate,up,down}_proj.trellis  I16 [k/16, n/16, 16 K]: exllamav3's tile record (any bits are a valid trellis)
  <P>.E.{gate,up,down}_proj.suh      F16 [k]; .svh F16 [n]
  <P>.E.{...}_proj.mul1 / .mcg       I32 scalar marker 0x83DCD12D / 0xCBAC1FED (neither: 3inst)
  <P> = model.language_model.layers.L.mlp.experts (trunk), mtp.layers.0.mlp.experts (the MTP head, layer index L =
  num_hidden_layers).

The experts here (hidden H = 256, expert width W = 128: gate / up are n = W out x k = H in, down n = H x k = W, so a
transposition shows):
  layer 0, expert 0   K=4 mul1      expert 1  K=3 mcg      expert 2  K=2 3inst (no marker)
  MTP head, expert 0  K=4 mul1
  layer 1 (hidden 128: each expert one defect, K=2 mul1 unless named):
    0 gate marker holds a wrong value        1 gate carries both markers        2 down has a .bias
    3 down trellis last dim 16 K + 8 (K=2.5) 4 up lacks its svh                 5 gate trellis tiles [k/16, n/16 - 1]
    6 down marker is F16, not I32            7 gate suh of length k - 64        8 gate trellis is I32
    9 valid (K=4 mul1: asked as K=3 or mcg)  10 up_proj absent
Run from anywhere: python3 tests/golden/gen_exl3_ckpt.py [OUTDIR]. The output is a function of the seed alone.
"""
from __future__ import annotations

import json
import os
import sys

import numpy as np
from safetensors.numpy import save_file

H, W = 256, 128
H1 = 128          # layer 1's hidden size (its experts only carry defects)
SEED = 20261202
MUL1, MCG = 0x83DCD12D, 0xCBAC1FED


def i32(v: int) -> np.ndarray:
    return np.array(v - (1 << 32) if v >= 1 << 31 else v, dtype=np.int32)


def proj(rng, k: int, n: int, bits: int, marker: str | None):
    t = {"trellis": rng.integers(-32768, 32768, size=(k // 16, n // 16, 16 * bits), dtype=np.int16),
         "suh": (rng.integers(0, 2, size=k) * 2 - 1).astype(np.float16),
         "svh": ((rng.integers(0, 2, size=n) * 2 - 1) / np.sqrt(k)).astype(np.float16)}
    if marker == "mul1":
        t["mul1"] = i32(MUL1)
    elif marker == "mcg":
        t["mcg"] = i32(MCG)
    return t


def expert(rng, bits: int, marker: str | None, h: int = H):
    return {"gate_proj": proj(rng, h, W, bits, marker), "up_proj": proj(rng, h, W, bits, marker),
            "down_proj": proj(rng, W, h, bits, marker)}


def build():
    rng = np.random.default_rng(SEED)
    trunk, mtp = "model.language_model.layers.%d.mlp.experts.%d", "mtp.layers.0.mlp.experts.%d"
    shard1, shard2 = {}, {}

    def put(dst, prefix, ex):
        for p, ts in ex.items():
            for name, v in ts.items():
                dst[f"{prefix}.{p}.{name}"] = v

    put(shard1, trunk % (0, 0), expert(rng, 4, "mul1"))
    put(shard1, trunk % (0, 1), expert(rng, 3, "mcg"))
    put(shard1, trunk % (0, 2), expert(rng, 2, None))
    put(shard1, mtp % 0, expert(rng, 4, "mul1"))
    for e in range(11):
        ex = expert(rng, 4 if e == 9 else 2, "mul1", H1)
        if e == 0:
            ex["gate_proj"]["mul1"] = i32(MUL1 ^ 1)
        elif e == 1:
            ex["gate_proj"]["mcg"] = i32(MCG)
        elif e == 2:
            ex["down_proj"]["bias"] = np.zeros(H1, np.float16)
        elif e == 3:
            ex["down_proj"]["trellis"] = rng.integers(-32768, 32768, size=(W // 16, H1 // 16, 40), dtype=np.int16)
        elif e == 4:
            del ex["up_proj"]["svh"]
        elif e == 5:
            ex["gate_proj"]["trellis"] = ex["gate_proj"]["trellis"][:, :-1].copy()
        elif e == 6:
            ex["down_proj"]["mul1"] = np.array(1.0, dtype=np.float16)
        elif e == 7:
            ex["gate_proj"]["suh"] = ex["gate_proj"]["suh"][:-64].copy()
        elif e == 8:
            ex["gate_proj"]["trellis"] = ex["gate_proj"]["trellis"].astype(np.int32)
        elif e == 10:
            del ex["up_proj"]
        put(shard2, trunk % (1, e), ex)
    return shard1, shard2


def write(outdir: str):
    os.makedirs(outdir, exist_ok=True)
    shard1, shard2 = build()
    files = {"model-00001-of-00002.safetensors": shard1, "model-00002-of-00002.safetensors": shard2}
    weight_map = {}
    for fname, tensors in files.items():
        save_file(tensors, os.path.join(outdir, fname), metadata={"format": "pt"})
        for name in tensors:
            weight_map[name] = fname
    total = sum(int(v.nbytes) for t in files.values() for v in t.values())
    with open(os.path.join(outdir, "model.safetensors.index.json"), "w") as f:
        json.dump({"metadata": {"total_size": total}, "weight_map": dict(sorted(weight_map.items()))}, f, indent=1)
        f.write("\n")
    config = {"architectures": ["Qwen3NextForCausalLM"], "model_type": "qwen3_next",
              "text_config": {"num_hidden_layers": 2, "hidden_size": H, "moe_intermediate_size": W,
                              "num_experts": 11, "num_experts_per_tok": 2},
              "quantization_config": {"quant_method": "exl3", "version": "0.0.7", "bits": 4, "head_bits": 6,
                                      "calibration": {"rows": 0, "cols": 0}}}
    with open(os.path.join(outdir, "config.json"), "w") as f:
        json.dump(config, f, indent=1)
        f.write("\n")


if __name__ == "__main__":
    write(sys.argv[1] if len(sys.argv) > 1 else os.path.join(os.path.dirname(os.path.abspath(__file__)), "exl3_ckpt"))
