#!/usr/bin/env python3
"""bench.py -- throughput of the EXL3 routed-expert decode layer on one MI355X.

One STEP is one routed-MoE layer in decode: 8 tokens (2 sequences x 4 speculative positions) through 512 experts at
4 bpw (gate/up 2048 -> 2 x 512, down 512 -> 2048, codebook mul1), router softmax -> top-10 -> renormalised, as ONE
moe_exl3_gate_up_down launch of libexl3c4.so (prep, gate_up with the h_rot epilogue, down). The router, the scatter and
the gather are the engine's ops in the reference (include/exl3_abi.h:90-118) and run outside the timed region.

Measurement hygiene: all experts of `--layers` independent layers are resident in HBM (about 0.8 GB a layer) and every
step uses the next layer and the next of `--draws` routing draws, so the ~120 MB a step reads was not read in the
previous several hundred MB (MI355X's 256 MB Infinity Cache). The timed steps are captured once into a HIP graph and
replayed, so host launch cost does not pace the GPU. Inputs are resident before the timed region starts.

Prints ONE JSON line. `value` is tokens/s of the layer; `roofline` is the dominant kernel's (gate_up's trellis-decode
GEMV) achieved packed-weight bandwidth against the 8 TB/s HBM peak, its duration timed live by events the dispatch
itself stamps; `cpu_baseline` times the CPU oracle (this repository's C restatement of the reference's exl3ref, one
thread) on a bounded sample of the same workload.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (ROOT, os.path.join(ROOT, "radiance-exl3_amd"), os.path.join(ROOT, "oracle"), os.path.join(ROOT, "tests")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

import numpy as np

H, W, E, TOP_K, M, BITS, CB = 2048, 512, 512, 10, 8, 4, "mul1"
HBM_PEAK_GBPS = 8000.0
GU_CODE_BYTES = 2 * W * H * BITS // 8            # one expert's gate_up codes (the GEMV's weight stream)
EXPERT_BYTES = 3 * W * H * BITS // 8 + 2 * (H + H + 2 * W) + 2 * (W + H)   # codes + scale planes: 1,588,224 at K=4


def build_layers(torch, n_layers, seed):
    """Stored records drawn uniformly (a bijection of uniformly random canonical planes) and scales on the device."""
    import exl3c4
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    layers = []
    gu_bytes, dn_bytes = 2 * W * H * BITS // 8, H * W * BITS // 8
    for _ in range(n_layers):
        L = {}
        L["gu_codes"] = torch.randint(0, 256, (E, gu_bytes), dtype=torch.uint8, device="cuda", generator=g)
        L["dn_codes"] = torch.randint(0, 256, (E, dn_bytes), dtype=torch.uint8, device="cuda", generator=g)

        def signs(n, mag):
            s = torch.randint(0, 2, (E, n), device="cuda", generator=g).to(torch.float16) * 2 - 1
            return (s * mag).contiguous().view(torch.int16)
        L["suh"], L["suh1"] = signs(H, 1.0), signs(H, 1.0)
        L["svh"] = signs(2 * W, 1.0 / np.sqrt(H))
        L["dn_suh"], L["dn_svh"] = signs(W, 1.0), signs(H, 1.0 / np.sqrt(W))
        L["gu_cls"] = exl3c4.make_class(2 * W, H, codes=L["gu_codes"], suh=L["suh"], suh1=L["suh1"], svh=L["svh"],
                                        dn_suh=L["dn_suh"])
        L["dn_cls"] = exl3c4.make_class(H, W, codes=L["dn_codes"], svh=L["dn_svh"])
        layers.append(L)
    return layers


def build_draws(torch, n_draws, seed):
    import exl3c4_synth as syn
    rng = np.random.default_rng(seed)
    draws = []
    for _ in range(n_draws):
        ids, w = syn.router_topk(rng.standard_normal((M, E)).astype(np.float32), TOP_K)
        st, off = syn.moe_scatter(ids, E)
        x = rng.standard_normal((M, H)).astype(np.float16)
        draws.append({"ids": ids, "w": w, "n_live": int(np.count_nonzero(np.diff(off))),
                      "sorted_tok": torch.from_numpy(st).cuda(), "off": torch.from_numpy(off).cuda(),
                      "x": torch.from_numpy(x.view(np.int16)).cuda(), "x_np": x, "st_np": st, "off_np": off})
    return draws


def cpu_baseline(draw, max_experts, seed):
    """The oracle's gate_up_down (scalar, one thread) on the live experts of one routing draw -- or the first
    `max_experts` of them, the time scaled to all -- with freshly drawn canonical planes of the same geometry."""
    import exl3c4_synth as syn
    import oracle
    rng = np.random.default_rng(seed)
    off, st = draw["off_np"], draw["st_np"]
    live = [e for e in range(E) if off[e + 1] > off[e]]
    take = live[:max_experts]
    # the sample: the routing restricted to the taken experts, renumbered 0..n-1 (the same rows, the same work)
    keep_rows = np.concatenate([np.arange(off[e], off[e + 1]) for e in take])
    sub_st = st[keep_rows].astype(np.int32)
    sub_off = np.zeros(len(take) + 1, np.int32)
    sub_off[1:] = np.cumsum([off[e + 1] - off[e] for e in take])
    n = len(take)
    gu = {"rows": 2 * W, "cols": H, "codes": syn.random_codes(rng, 2 * W, H, BITS, n),
          "suh": syn.sign_scales(rng, H, 1.0, n), "suh1": syn.sign_scales(rng, H, 1.0, n),
          "svh": syn.sign_scales(rng, 2 * W, 1 / np.sqrt(H), n), "dn_suh": syn.sign_scales(rng, W, 1.0, n)}
    dn = {"rows": H, "cols": W, "codes": syn.random_codes(rng, H, W, BITS, n),
          "suh": gu["dn_suh"], "svh": syn.sign_scales(rng, H, 1 / np.sqrt(W), n)}
    x = draw["x_np"].view(np.uint16)
    oracle.lib()
    t0 = time.perf_counter()
    oracle.run_gate_up_down([gu], [dn], BITS, CB, x, sub_st, sub_off, TOP_K)
    dt = time.perf_counter() - t0
    t_layer = dt * len(live) / n
    return {"value": round(M / t_layer, 3), "unit": "tokens/s", "cores": 1, "kind": "port",
            "sample": (f"{n} of the {len(live)} live experts of one decode layer step (8 tokens, top-10, K=4 mul1), "
                       f"oracle/exl3_oracle.c gate_up_down on 1 thread: {dt:.2f} s, scaled x{len(live) / n:.2f} "
                       f"to the whole layer")}


def read_traffic():
    """HBM bytes per launch of the dominant kernel from the committed rocprofv3 --pmc summary, if there is one."""
    p = os.path.join(ROOT, "profiles", "traffic_k_gu_decode.json")
    if not os.path.exists(p):
        return None
    with open(p) as f:
        return json.load(f).get("bytes_per_launch")


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--layers", type=int, default=8)
    ap.add_argument("--draws", type=int, default=8)
    ap.add_argument("--cpu-experts", type=int, default=24, help="live experts in the CPU-baseline sample (0: skip)")
    ap.add_argument("--seed", type=int, default=20261013)
    ap.add_argument("--copy-probe", type=int, default=0, metavar="BYTES",
                    help="only run 20 plain device-to-device copies of BYTES (the HBM-counter calibration) and exit")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py runs on ONE GPU: this build has no multi-GPU path (asked for --gpus {args.gpus}).",
              file=sys.stderr)
        sys.exit(2)

    import torch
    if args.copy_probe > 0:
        src = torch.empty(args.copy_probe, dtype=torch.uint8, device="cuda").fill_(1)
        dst = torch.empty_like(src)
        for _ in range(20):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_probe_bytes": args.copy_probe, "copies": 20}), flush=True)
        return
    import exl3c4
    exl3c4.lib()
    torch.cuda.set_device(0)
    layers = build_layers(torch, args.layers, args.seed)
    draws = build_draws(torch, args.draws, args.seed + 1)
    T = M * TOP_K
    y = torch.zeros((T, H), dtype=torch.int16, device="cuda")
    ops = []
    for s in range(max(args.layers, args.draws)):
        L, D = layers[s % args.layers], draws[s % args.draws]
        ops.append(exl3c4.make_op(exl3c4.GU_DN, BITS, CB, [L["gu_cls"]], D["x"], D["sorted_tok"], D["off"], y, M,
                                  TOP_K, dn=[L["dn_cls"]]))
    scratch = exl3c4.alloc_scratch(ops[0])
    stream = torch.cuda.current_stream()

    def step(i):
        rc = exl3c4.launch(ops[i % len(ops)], scratch, stream)
        if rc:
            raise RuntimeError(f"launch: {exl3c4.STATUS.get(rc, rc)}")

    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()

    # the timed region: K steps captured once as a HIP graph, replayed
    g = torch.cuda.CUDAGraph()
    cap = torch.cuda.Stream()
    cap.wait_stream(stream)
    with torch.cuda.stream(cap):
        with torch.cuda.graph(g, stream=cap):
            for i in range(args.steps):
                rc = exl3c4.launch(ops[i % len(ops)], scratch, torch.cuda.current_stream())
                if rc:
                    raise RuntimeError(f"launch under capture: {exl3c4.STATUS.get(rc, rc)}")
    stream.wait_stream(cap)
    g.replay()                                    # one untimed replay (first-replay costs)
    torch.cuda.synchronize()
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0.record()
    g.replay()
    t1.record()
    torch.cuda.synchronize()
    ms = t0.elapsed_time(t1)
    ms_step = ms / args.steps
    tokens_s = M * args.steps / (ms / 1e3)
    live = [draws[i % args.draws]["n_live"] for i in range(args.steps)]
    layer_bytes = float(np.mean(live)) * EXPERT_BYTES
    layer_gbps = layer_bytes / (ms_step * 1e-3) / 1e9

    # the dominant kernel (gate_up's GEMM), live: events stamped around its own dispatch, eager steps queued behind a
    # short spin so that they run back to back as in the timed region (no host gaps between them)
    evs = [(exl3c4.Event(), exl3c4.Event()) for _ in range(args.steps)]
    torch.cuda._sleep(int(2e6 + 2e5 * args.steps))
    for i in range(args.steps):
        a, b = evs[i]
        rc = exl3c4.launch_timed(ops[i % len(ops)], scratch, exl3c4.K_GATE_UP, a, b, stream)
        if rc:
            raise RuntimeError(f"timed launch: {exl3c4.STATUS.get(rc, rc)}")
    torch.cuda.synchronize()
    durs = np.array([exl3c4.elapsed_ms(a, b) for a, b in evs])      # ms
    gemv_bytes = np.array(live, dtype=np.float64) * GU_CODE_BYTES
    gemv_gbps = float(np.mean(gemv_bytes) / (np.mean(durs) * 1e-3) / 1e9)

    cpu = None
    if args.cpu_experts > 0:
        cpu = cpu_baseline(draws[0], args.cpu_experts, args.seed + 2)

    out = {
        "metric": "MoE-layer tokens/s + packed-weight GB/s (% HBM peak) decode; prefill % MFMA peak",
        "value": round(tokens_s, 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic",
        "config": {"workload": "configs[2]: routed MoE layer decode, 512 experts (gate/up 2048->2x512, down "
                               "512->2048) at 4 bpw mul1, 8 tokens, router softmax top-10 renormalised, one "
                               "moe_exl3_gate_up_down launch per step",
                   "layers_resident": args.layers, "routing_draws": args.draws,
                   "mean_live_experts": round(float(np.mean(live)), 2)},
        "packed_weight_GBps": round(layer_gbps, 1),
        "hbm_frac": round(layer_gbps / HBM_PEAK_GBPS, 4),
        "roofline": {"bound": "hbm", "achieved": round(gemv_gbps, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": round(gemv_gbps / HBM_PEAK_GBPS, 4), "traffic": read_traffic(),
                     "kernel": "k_gu<4,mul1> (gate_up GEMM)", "avg_us": round(float(np.mean(durs)) * 1e3, 3),
                     "bytes_per_launch": round(float(np.mean(gemv_bytes)))},
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
