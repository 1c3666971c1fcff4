#!/usr/bin/env python3
"""bench.py -- throughput of the EXL3 routed-expert decode layer on one MI355X; with
--config 2, 4 or 5 the single expert, the prefill layer or the 48-layer decode stack instead.

One STEP is one routed-MoE layer in decode, the whole layer on the device: 8 tokens (2 sequences x 4 speculative
positions) through 512 experts at 4 bpw (gate/up 2048 -> 2 x 512, down 512 -> 2048, codebook mul1): the router
(softmax over N(0,1) logits -> top-10 -> renormalised) with the stable scatter by expert, then ONE
moe_exl3_gate_up_down launch of libexl3c4.so whose single kernel also does moe_gather (the weighted sum in f32, cast to
f16). The same step with the gather as its own dispatch, and the op alone, are timed beside it.

Measurement hygiene: all experts of `--layers` independent layers are resident in HBM (about 0.8 GB a layer) and every
step uses the next layer and the next of `--draws` routing draws, so the ~120 MB a step reads was not read in the
previous several hundred MB (MI355X's 256 MB Infinity Cache). The timed steps are captured once into a HIP graph and
replayed, so host launch cost does not pace the GPU. Inputs are resident before the timed region starts.

Prints ONE JSON line. `value` is tokens/s of the layer; `roofline` is the dominant kernel's (gate_up_down's single
kernel) achieved packed-weight bandwidth against the 8 TB/s HBM peak, its duration timed live by events the dispatch
itself stamps, on its live experts' codes and scale planes; `roofline_valu` the same kernel against the VALU issue
rate its trellis decode is bound by (its counted instructions); `prefill` the prefill layer (configs[3]: 2048 tokens,
Zipf routing) and `stack` the 48-layer mixed-K decode stack, both measured in the same run;
`peaks_measured` the box's own ceilings from this library's calibration kernels (libexl3c4_calib.so: HBM stream read,
VALU issue rate and clock, f16 MFMA rate); `cpu_baseline` times the CPU oracle (this repository's C restatement of
the reference's exl3ref) on the same workload, on one thread and on the box's cores, and configs[0]'s single linear.
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
CODE_BYTES = 3 * W * H * BITS // 8               # one expert's gate_up and down codes
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
        logits = rng.standard_normal((M, E)).astype(np.float32)
        ids, w = syn.router_topk(logits, TOP_K)
        st, off = syn.moe_scatter(ids, E)
        x = rng.standard_normal((M, H)).astype(np.float16)
        draws.append({"ids": ids, "w": w, "n_live": int(np.count_nonzero(np.diff(off))),
                      "sorted_tok": torch.from_numpy(st).cuda(), "off": torch.from_numpy(off).cuda(),
                      "logits": torch.from_numpy(logits).cuda(),
                      "x": torch.from_numpy(x.view(np.int16)).cuda(), "x_np": x, "st_np": st, "off_np": off})
    return draws


def cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def _median_s(fn, runs=3):
    """One untimed warm run, then the median of `runs` timed runs (seconds, CLOCK_MONOTONIC via perf_counter)."""
    fn()
    ts = []
    for _ in range(runs):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    return float(np.median(ts))


def cpu_baseline(draw, max_experts, seed, one_thread_experts=12):
    """The oracle's gate_up_down (this repository's C restatement of exl3ref, oracle/exl3_oracle.c) on the live experts
    of one routing draw, with freshly drawn canonical planes of the same geometry: on the box's cores over every live
    expert (OpenMP over experts; the outputs do not depend on the count), and on one thread over the first
    `one_thread_experts` of them, its time scaled to the layer. Each figure is the median of 3 runs after one warm run.
    Beside them, configs[0]: the CPU single linear (K_in 2048 -> N_out 512, K=4 mul1, one token), the oracle's down op
    on one expert -- the input rotation, the W_hat decode, the ascending-k f32 GEMV, had128 x svh -- on one thread."""
    import exl3c4_synth as syn
    import oracle
    rng = np.random.default_rng(seed)
    off, st = draw["off_np"], draw["st_np"]
    live = [e for e in range(E) if off[e + 1] > off[e]][:max_experts]

    def sample(take):
        # the routing restricted to the taken experts, renumbered 0..n-1 (the same rows, the same work)
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
        return gu, dn, sub_st, sub_off
    x = draw["x_np"].view(np.uint16)
    oracle.lib()
    cores = oracle.default_threads()
    gu, dn, sub_st, sub_off = sample(live)
    oracle.set_threads(cores)
    t_all = _median_s(lambda: oracle.run_gate_up_down([gu], [dn], BITS, CB, x, sub_st, sub_off, TOP_K))
    take1 = live[:one_thread_experts]
    gu1, dn1, st1, off1 = sample(take1)
    oracle.set_threads(1)
    t_one = _median_s(lambda: oracle.run_gate_up_down([gu1], [dn1], BITS, CB, x, st1, off1, TOP_K))
    scale1 = len(live) / len(take1)
    # one linear [N_out 512, K_in 2048] at K=4 mul1, one token (sorted row 0 -> expert 0)
    lin = {"rows": W, "cols": H, "codes": syn.random_codes(rng, W, H, BITS, 1),
           "suh": syn.sign_scales(rng, H, 1.0, 1), "svh": syn.sign_scales(rng, W, 1 / np.sqrt(H), 1)}
    x1 = syn.normal_f16(rng, (1, H)).view(np.uint16)
    t_lin = _median_s(lambda: oracle.run_op(oracle.OP_DOWN, [lin], BITS, CB, x1, np.zeros(1, np.int32),
                                            np.array([0, 1], np.int32), 1))
    oracle.set_threads(cores)
    return {"value": round(M / t_all, 3), "unit": "tokens/s", "cores": cores, "kind": "port",
            "value_1thread": round(M / (t_one * scale1), 3), "nproc": os.cpu_count(), "cpu_model": cpu_model(),
            "sample": (f"one decode layer step (8 tokens, top-10, K=4 mul1), oracle/exl3_oracle.c gate_up_down, "
                       f"median of 3 after a warm run: all {len(live)} live experts on {cores} threads "
                       f"({t_all:.2f} s); the first {len(take1)} on 1 thread ({t_one:.2f} s, scaled x{scale1:.2f})"),
            "configs0_linear": {"ms": round(t_lin * 1e3, 2), "threads": 1,
                                "what": "configs[0]: one EXL3 linear 2048 -> 512 at K=4 mul1, 1 token: input rotation, "
                                        "W_hat decode of 1,048,576 weights, ascending-k f32 GEMV, had128 x svh "
                                        "(the oracle's down op), median of 3 after a warm run"}}


def read_traffic(name):
    """HBM bytes per launch of the dominant kernel from the committed rocprofv3 --pmc summary
    (profiles/traffic_<name>.json), if there is one."""
    p = os.path.join(ROOT, "profiles", f"traffic_{name}.json")
    if not os.path.exists(p):
        return None
    with open(p) as f:
        return json.load(f).get("bytes_per_launch")


WARM_MS = 10.0       # device time of untimed replays queued right ahead of the timed one


def timed_graph(torch, launch_step, steps, warmup):
    """Warm up eagerly, capture `steps` steps into one HIP graph, replay once untimed, then time one replay with events
    around it. Returns ms for the whole replay.

    The timed replay follows untimed replays of the same graph queued right ahead of it (at least WARM_MS of device
    time, without a host synchronisation in between): the device is running the same steps when the start event
    fires, at the clocks it holds under this load, and the host's submission of the timed replay overlaps them. The
    events time exactly the `steps` steps of the last replay. (From an idle device the first milliseconds of a replay
    run while the clocks ramp up and behind the host's hand-over of the graph's first kernels: measured on the
    decode layer, a replay of 20 steps then read 53-55 us a step against 50 for a replay of 200; behind 2 ms of warm
    replays 53, behind 10 ms 50.2-50.4, the 200-step figure, which the warm replays leave unchanged.)"""
    stream = torch.cuda.current_stream()
    for i in range(warmup):
        launch_step(i, stream)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    cap = torch.cuda.Stream()
    cap.wait_stream(stream)
    with torch.cuda.stream(cap):
        with torch.cuda.graph(g, stream=cap):
            for i in range(steps):
                launch_step(i, torch.cuda.current_stream())
    stream.wait_stream(cap)
    w0, w1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    w0.record()
    g.replay()                                    # one untimed replay (first-replay costs), timed to size the warm-up
    w1.record()
    torch.cuda.synchronize()
    n_warm = max(1, int(np.ceil(WARM_MS / max(w0.elapsed_time(w1), 1e-3))))
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    for _ in range(n_warm):
        g.replay()
    t0.record()
    g.replay()
    t1.record()
    torch.cuda.synchronize()
    return t0.elapsed_time(t1)


def kernel_ms(torch, exl3c4, ops, scratch, kernel, n):
    """Average duration (ms) of one kernel of the op sequence over n eager launches, timed by start/stop events
    around its own dispatch; the launches are queued behind a short spin so that they run back to back."""
    evs = [(exl3c4.Event(), exl3c4.Event()) for _ in range(n)]
    stream = torch.cuda.current_stream()
    torch.cuda._sleep(int(2e6 + 2e5 * n))
    for i in range(n):
        rc = exl3c4.launch_timed(ops[i % len(ops)], scratch, kernel, evs[i][0], evs[i][1], stream)
        if rc:
            raise RuntimeError(f"timed launch: {exl3c4.STATUS.get(rc, rc)}")
    torch.cuda.synchronize()
    return np.array([exl3c4.elapsed_ms(a, b) for a, b in evs])


def check_rc(exl3c4, rc):
    if rc:
        raise RuntimeError(f"launch: {exl3c4.STATUS.get(rc, rc)}")


def common(args, ms, steps, value, unit, workload, extra=None):
    out = {"metric": "MoE-layer tokens/s + packed-weight GB/s (% HBM peak) decode; prefill % MFMA peak",
           "value": round(value, 1), "unit": unit, "n_gpus": 1, "steps": steps, "warmup": args.warmup,
           "ms_per_step": round(ms / steps, 5), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
           "dtype": "f16", "data": "synthetic", "config": {"workload": workload}}
    if extra:
        out["config"].update(extra)
    return out


# ------------------------------------------------------------------------------------------ decode layer
def run_decode_layer(args, torch, exl3c4):
    """A step is the whole layer on the device: router_topk_scatter on the draw's logits (softmax over the 512 experts,
    top-10, renormalised; the stable scatter), one gate_up_down launch, and moe_gather (the weighted sum in f32, cast
    to f16), the gather riding in gate_up_down's kernel (exl3c4_launch_gather); the same step with the gather as its
    own dispatch is timed beside it."""
    layers = build_layers(torch, args.layers, args.seed)
    draws = build_draws(torch, args.draws, args.seed + 1)
    T = M * TOP_K
    y = torch.zeros((T, H), dtype=torch.int16, device="cuda")
    out_t = torch.zeros((M, H), dtype=torch.int16, device="cuda")
    ids = torch.zeros((M, TOP_K), dtype=torch.int32, device="cuda")
    w = torch.zeros((M, TOP_K), dtype=torch.float32, device="cuda")
    st_d = torch.zeros((T,), dtype=torch.int32, device="cuda")
    off_d = torch.zeros((E + 1,), dtype=torch.int32, device="cuda")
    row_of = torch.zeros((T,), dtype=torch.int32, device="cuda")
    n = max(args.layers, args.draws)
    layer_ops, ops = [], []
    for s in range(n):
        L, D = layers[s % args.layers], draws[s % args.draws]
        layer_ops.append(exl3c4.make_op(exl3c4.GU_DN, BITS, CB, [L["gu_cls"]], D["x"], st_d, off_d, y, M, TOP_K,
                                        dn=[L["dn_cls"]]))
        ops.append(exl3c4.make_op(exl3c4.GU_DN, BITS, CB, [L["gu_cls"]], D["x"], D["sorted_tok"], D["off"], y, M,
                                  TOP_K, dn=[L["dn_cls"]]))
    scratch = exl3c4.alloc_scratch(ops[0])
    # gate_up_down's counter block: zeroed once here, left zeroed by every launch (exl3c4_launch_ctr)
    ctr = torch.zeros(max(exl3c4.ctr_bytes(ops[0]), 256), dtype=torch.uint8, device="cuda")

    def layer_step(i, stream):
        D = draws[i % n % args.draws]
        check_rc(exl3c4, exl3c4.router_topk_scatter(D["logits"], TOP_K, True, ids, w, st_d, off_d, None, row_of,
                                                    stream))
        check_rc(exl3c4, exl3c4.launch_gather(layer_ops[i % n], scratch, ctr, w, row_of, out_t, stream))

    def layer_step_separate(i, stream):
        D = draws[i % n % args.draws]
        check_rc(exl3c4, exl3c4.router_topk_scatter(D["logits"], TOP_K, True, ids, w, st_d, off_d, None, row_of,
                                                    stream))
        check_rc(exl3c4, exl3c4.launch_ctr(layer_ops[i % n], scratch, ctr, stream))
        check_rc(exl3c4, exl3c4.moe_gather(y, True, w, row_of, out_t, stream))
    if args.op_only:                                  # for a profiler's run: the op graph alone
        ms_op = timed_graph(torch, lambda i, st: check_rc(exl3c4, exl3c4.launch_ctr(ops[i % n], scratch, ctr, st)),
                            args.steps, args.warmup)
        return {"op_only": True, "op_us": round(ms_op / args.steps * 1e3, 2), "steps": args.steps}
    ms_sep = timed_graph(torch, layer_step_separate, args.steps, args.warmup)
    ms = timed_graph(torch, layer_step, args.steps, args.warmup)
    ms_op = timed_graph(torch, lambda i, st: check_rc(exl3c4, exl3c4.launch_ctr(ops[i % n], scratch, ctr, st)),
                        args.steps, args.warmup)
    ms_step = ms / args.steps
    live = [draws[i % n % args.draws]["n_live"] for i in range(args.steps)]
    st = int(ctr[:4].cpu().numpy().view(np.int32)[0])
    if st or int(torch.count_nonzero(ctr)):
        raise RuntimeError(f"gate_up_down's single kernel left status {st} or a nonzero counter block")
    layer_gbps = float(np.mean(live)) * EXPERT_BYTES / (ms_step * 1e-3) / 1e9
    one = T >= exl3c4.GD_FUSE_MIN_T           # gate_up_down runs as one kernel: that kernel is the one timed
    durs = kernel_ms(torch, exl3c4, ops, scratch, exl3c4.K_GATE_UP_DOWN if one else exl3c4.K_GATE_UP, args.steps)
    # the kernel's average launch duration as the layer runs it: the op graph's replay, back-to-back launches of the
    # one kernel (a caller's zeroed counter block, no fill), events around the replay; beside it the eager launches'
    # own event pairs (each dispatch behind a counter fill, stamped at its start and end)
    avg_ms = ms_op / args.steps if one else float(np.mean(durs))
    # the kernel's algorithmic bytes: its live experts' packed codes and scale planes (perfmoe's definition)
    gemv_bytes = np.array(live, dtype=np.float64) * (EXPERT_BYTES if one else GU_CODE_BYTES)
    gemv_gbps = float(np.mean(gemv_bytes) / (avg_ms * 1e-3) / 1e9)
    kname = "k_gd_decode" if one else "k_gu_decode"
    # the memory floor of the same bytes: the step's live experts' planes read the way the kernel reads them
    floor = extent_read_floor(torch, layers, draws, n) if args.peaks else None
    cpu = cpu_baseline(draws[0], args.cpu_experts, args.seed + 2) if args.cpu_experts > 0 else None
    out = common(args, ms, args.steps, M * args.steps / (ms / 1e3), "tokens/s",
                 "configs[2]: routed MoE layer decode, 512 experts (gate/up 2048->2x512, down 512->2048) at 4 bpw "
                 "mul1, 8 tokens; a step is the whole layer on the device: router_topk_scatter (softmax over N(0,1) "
                 "logits, top-10, renormalised, stable scatter), one moe_exl3_gate_up_down launch with moe_gather (f32 "
                 "weighted sum, f16 out) inside its kernel (exl3c4_launch_gather)",
                 {"layers_resident": args.layers, "routing_draws": args.draws,
                  "mean_live_experts": round(float(np.mean(live)), 2)})
    out.update({
        "op_us": round(ms_op / args.steps * 1e3, 2),              # the gate_up_down launch alone, graph replay
        "step_us_gather_separate": round(ms_sep / args.steps * 1e3, 2),   # the step with moe_gather dispatched alone
        "packed_weight_GBps": round(layer_gbps, 1),
        "hbm_frac": round(layer_gbps / HBM_PEAK_GBPS, 4),
        "roofline": {"bound": "hbm", "achieved": round(gemv_gbps, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": round(gemv_gbps / HBM_PEAK_GBPS, 4), "traffic": read_traffic(kname),
                     "kernel": "k_gd<4,mul1> (gate_up_down, one kernel)" if one else "k_gu<4,mul1> (gate_up GEMM)",
                     "avg_us": round(avg_ms * 1e3, 3),
                     "avg_us_how": ("graph replay of the op alone: back-to-back launches of its one kernel, events "
                                    "around the replay" if one else "event pairs around each eager dispatch"),
                     "avg_us_eager": round(float(np.mean(durs)) * 1e3, 3),
                     "bytes_per_launch": round(float(np.mean(gemv_bytes))),
                     "bytes_what": "live experts x (packed codes + suh, suh1, svh, dn_suh, dn_svh): 1,588,224 B each"},
        "roofline_valu": valu_roofline(float(np.mean(live)), avg_ms * 1e-3),
        "cpu_baseline": cpu,
    })
    if floor:
        out["roofline"]["extent_read_floor"] = floor
    return out


# The decode loop's VALU work, read from the gfx950 assembly of k_gd<4,mul1> (the same loop body in k_gu / k_dn): an
# iteration of two steps -- each step a wave's 32-column strip over 64 k, 2048 weights -- issues 253 VALU instructions
# (64 v_pk_mul_lo_u16, 64 v_mad_u32_u16, 32 v_sad_u8, 32 v_sad_hi_u8, 32 v_pk_fma_f16, 18 v_alignbit_b32, 6 v_perm_b32,
# 5 others) and 8 MFMAs. The kernel's whole issue (its start-ups, epilogues, gather) is counted by SQ_INSTS_VALU in
# profiles/valu_k_gd_decode.json when that profile exists, and the line uses the count.
VALU_PER_STEP, WEIGHTS_PER_STEP = 126.5, 2048
# A SIMD issues one wave64 VALU instruction each 4 cycles; 1024 SIMDs at MI355X's 2.4 GHz peak engine clock.
VALU_PEAK_GINSTR = 1024 * 2.4 / 4


def read_counted_valu():
    """SQ_INSTS_VALU a k_gd dispatch and the mean live experts of the run it was counted on (the committed rocprofv3
    --pmc summary), or None."""
    p = os.path.join(ROOT, "profiles", "valu_k_gd_decode.json")
    if not os.path.exists(p):
        return None
    with open(p) as f:
        return json.load(f)


def valu_roofline(live, seconds, peak_measured=None):
    """The decode kernel against the VALU issue roofline: its wave instructions over its duration. The instructions
    are the counted SQ_INSTS_VALU a dispatch (scaled to this run's live experts) when the profile is committed, else
    the loop's count alone."""
    c = read_counted_valu()
    if c:
        instr = float(c["sq_insts_valu_per_dispatch"]) * live / float(c["mean_live_experts"])
        how = (f"SQ_INSTS_VALU a dispatch ({c['sq_insts_valu_per_dispatch']:.4g} at {c['mean_live_experts']} live "
               f"experts, profiles/valu_k_gd_decode.json), scaled to this run's {live:.2f}")
    else:
        instr = live * 3 * W * H / WEIGHTS_PER_STEP * VALU_PER_STEP
        how = "the decode loop's 126.5 instructions a 2048-weight step only (no counter profile committed)"
    achieved = instr / seconds / 1e9
    out = {"bound": "valu", "achieved": round(achieved, 1), "peak": VALU_PEAK_GINSTR, "unit": "G wave-instr/s",
           "frac": round(achieved / VALU_PEAK_GINSTR, 4), "instr_per_launch": round(instr),
           "floor_us": round(instr / VALU_PEAK_GINSTR / 1e3, 2), "instr_how": how}
    if peak_measured:
        out["peak_measured"] = peak_measured
        out["frac_measured"] = round(achieved / peak_measured, 4)
    return out


_calib = None


def calib():
    """libexl3c4_calib.so: this library's own stream-read, VALU-issue and MFMA kernels (the box's ceilings)."""
    global _calib
    if _calib is None:
        import ctypes as C
        _calib = C.CDLL(os.path.join(ROOT, "radiance-exl3_amd", "libexl3c4_calib.so"))
        f, p, i32, i64 = C.c_float, C.c_void_p, C.c_int32, C.c_int64
        _calib.exl3c4_calib_read.restype = f
        _calib.exl3c4_calib_read.argtypes = [p, i64, i32, p, i32, p]
        _calib.exl3c4_calib_read_runs.restype = f
        _calib.exl3c4_calib_read_runs.argtypes = [p, p, i32, i64, i32, p, i32, p]
        _calib.exl3c4_calib_valu.restype = f
        _calib.exl3c4_calib_valu.argtypes = [i32, i32, p, i32, p]
        _calib.exl3c4_calib_mfma.restype = f
        _calib.exl3c4_calib_mfma.argtypes = [i32, i32, p, i32, p]
    return _calib


def _ok_ms(ms, what):
    if ms <= 0:
        raise RuntimeError(f"{what}: calibration kernel failed ({ms})")
    return ms


def extent_read_floor(torch, layers, draws, n):
    """The decode kernel's bytes as a plain read: for each step's layer and draw, every live expert's gate_up and down
    codes read in 8 KiB runs (a wave a run, 1 KiB a step, two steps in flight: the decode kernels' access), all steps'
    extents in one launch each; the rate over the codes (GB/s), best of 8."""
    C = calib()
    st = torch.cuda.current_stream().cuda_stream
    sc = torch.zeros(64, dtype=torch.int32, device="cuda")
    rates = []
    for s in range(min(n, 8)):
        L, D = layers[s % len(layers)], draws[s % len(draws)]
        off = D["off_np"]
        ext = []
        for e in range(E):
            if off[e + 1] > off[e]:
                ext.append((L["gu_codes"][e].data_ptr(), L["gu_codes"][e].numel()))
                ext.append((L["dn_codes"][e].data_ptr(), L["dn_codes"][e].numel()))
        run = 8192
        assert all(b % run == 0 for _, b in ext)
        first = np.cumsum([0] + [b // run for _, b in ext[:-1]]).astype(np.int64)
        n_runs = int(sum(b // run for _, b in ext))
        ext_t = torch.from_numpy(np.array(ext, np.uint64).view(np.int64).reshape(-1)).cuda()
        first_t = torch.from_numpy(first).cuda()
        ms = _ok_ms(C.exl3c4_calib_read_runs(ext_t.data_ptr(), first_t.data_ptr(), len(ext), n_runs, run,
                                             sc.data_ptr(), 8, st), "read_runs")
        rates.append(sum(b for _, b in ext) / (ms * 1e-3) / 1e9)
    return {"GBps": round(float(np.median(rates)), 1), "unit": "GB/s on the codes",
            "how": "libexl3c4_calib.so k_read_runs: the step's live experts' codes in 8 KiB runs, a wave a run, "
                   "1 KiB a step, two in flight; median over the draws of the best of 8"}


def measured_peaks(torch):
    """What this box reaches, on this library's own kernels (libexl3c4_calib.so, event-timed, best of 8): HBM read (a
    4 GiB stream, 16-byte loads, four in flight a thread), the VALU issue rate of the trellis decode's own
    instructions (8 independent chains a wave, 4 to 8 waves a SIMD) and with it the engine clock under that load, and
    the f16 MFMA rate (v_mfma_f32_16x16x32_f16, 8 independent chains a wave); beside them torch's plain copy and fill
    and hipBLASLt's f16 GEMM (library work)."""
    C = calib()
    st = torch.cuda.current_stream().cuda_stream
    n = 1 << 30
    x = torch.ones(n, dtype=torch.float32, device="cuda")
    sc = torch.zeros(1 << 16, dtype=torch.int32, device="cuda")
    read = max(4.0 * n / (_ok_ms(C.exl3c4_calib_read(x.data_ptr(), 4 * n, blocks, sc.data_ptr(), 8, st),
                                 "read") * 1e-3) / 1e9 for blocks in (2048, 4096, 8192))

    def best_ms(fn, reps=8):
        fn()
        torch.cuda.synchronize()
        ts = []
        for _ in range(reps):
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record()
            fn()
            b.record()
            b.synchronize()
            ts.append(a.elapsed_time(b))
        return min(ts)
    y = torch.empty_like(x)
    copy_gbps = 8.0 * n / (best_ms(lambda: y.copy_(x)) * 1e-3) / 1e9
    fill_gbps = 4.0 * n / (best_ms(lambda: y.fill_(1.0)) * 1e-3) / 1e9          # write-only: k_rot's xr traffic
    del x, y
    rounds = 2000
    valu = []
    for wg_per_cu in (4, 8):              # 4 or 8 waves a SIMD
        blocks = 256 * wg_per_cu
        ms = _ok_ms(C.exl3c4_calib_valu(blocks, rounds, sc.data_ptr(), 8, st), "valu")
        valu.append(blocks * 4 * rounds * 56 / (ms * 1e-3) / 1e9)
    valu_g = max(valu)
    mfma = []
    for wg_per_cu in (4, 8):
        blocks = 256 * wg_per_cu
        ms = _ok_ms(C.exl3c4_calib_mfma(blocks, rounds, sc.data_ptr(), 8, st), "mfma")
        mfma.append(blocks * 4 * rounds * 8 * 16 * 16 * 32 * 2 / (ms * 1e-3) / 1e12)
    m = 8192
    g = torch.Generator(device="cuda").manual_seed(1)
    a = torch.randn(m, m, device="cuda", dtype=torch.float16, generator=g)
    b = torch.randn(m, m, device="cuda", dtype=torch.float16, generator=g)
    gemm_tflops = 2.0 * m ** 3 / (best_ms(lambda: torch.matmul(a, b), 6) * 1e-3) / 1e12
    del a, b
    torch.cuda.empty_cache()
    return {"hbm_read_GBps": round(read, 1), "hbm_copy_GBps": round(copy_gbps, 1), "hbm_fill_GBps": round(fill_gbps, 1),
            "valu_Ginstr_s": round(valu_g, 1), "valu_clock_GHz": round(valu_g * 4 / 1024, 3),
            "mfma_f16_TFLOPs": round(max(mfma), 1), "fp16_gemm_TFLOPs": round(gemm_tflops, 1),
            "how": ("best of 8 event-timed launches: libexl3c4_calib.so k_read over 4 GiB (hbm_read), k_valu (the "
                    "mul1 pair's 7 instructions x 8 chains a wave; clock = rate x 4 cycles / 1024 SIMDs), k_mfma "
                    "(v_mfma_f32_16x16x32_f16 x 8 chains a wave); torch copy_ of 4 GiB (read + write bytes); torch fill_ "
                    "of 4 GiB (write-only); "
                    "torch.matmul f16 8192^3 (hipBLASLt)")}


def add_measured(roofline, peak):
    """The roofline's fraction of what the box measured (peak_measured) beside its fraction of the spec peak."""
    if roofline is not None and peak:
        roofline["peak_measured"] = peak
        roofline["frac_measured"] = round(roofline["achieved"] / peak, 4)


# ------------------------------------------------------------------------------------------ one expert
def run_single_expert(args, torch, exl3c4):
    """One SwiGLU expert (gate/up 2048 -> 2 x 512, down 512 -> 2048) at K 3, 4, 5 and m 1, 4, 16 tokens, top_k 1: one
    gate_up_down launch a step; 64 copies of the expert resident, a different one each step (no cache reuse)."""
    copies, res = 64, []
    for bits in (3, 4, 5):
        g = torch.Generator(device="cuda")
        g.manual_seed(args.seed + bits)
        gu = torch.randint(0, 256, (copies, 2 * W * H * bits // 8), dtype=torch.uint8, device="cuda", generator=g)
        dn = torch.randint(0, 256, (copies, H * W * bits // 8), dtype=torch.uint8, device="cuda", generator=g)

        def signs(e, n, mag):
            s = torch.randint(0, 2, (e, n), device="cuda", generator=g).to(torch.float16) * 2 - 1
            return (s * mag).contiguous().view(torch.int16)
        suh, suh1, svh = signs(copies, H, 1.0), signs(copies, H, 1.0), signs(copies, 2 * W, 1 / np.sqrt(H))
        dsuh, dsvh = signs(copies, W, 1.0), signs(copies, H, 1 / np.sqrt(W))
        for m in (1, 4, 16):
            x = torch.randn((m, H), device="cuda", generator=g).to(torch.float16).view(torch.int16)
            st = torch.arange(m, dtype=torch.int32, device="cuda")
            offs = []
            for j in range(copies):        # every row to expert j (of `copies`), the others empty
                o = np.zeros(copies + 1, np.int32)
                o[j + 1:] = m
                offs.append(torch.from_numpy(o).cuda())
            y = torch.zeros((m, H), dtype=torch.int16, device="cuda")
            gcls = exl3c4.make_class(2 * W, H, codes=gu, suh=suh, suh1=suh1, svh=svh, dn_suh=dsuh)
            dcls = exl3c4.make_class(H, W, codes=dn, svh=dsvh)
            ops = [exl3c4.make_op(exl3c4.GU_DN, bits, CB, [gcls], x, st, offs[j], y, m, 1, dn=[dcls])
                   for j in range(copies)]
            scratch = exl3c4.alloc_scratch(ops[0])
            steps = args.steps
            ms = timed_graph(torch, lambda i, s_: check_rc(exl3c4, exl3c4.launch(ops[i % copies], scratch, s_)),
                             steps, args.warmup)
            us = ms / steps * 1e3
            byts = 393216 * bits + 15360
            res.append({"bits": bits, "m": m, "us": round(us, 2), "GBps": round(byts / (us * 1e-6) / 1e9, 1),
                        "tokens_s": round(m / (us * 1e-6), 1)})
    k4m16 = [r for r in res if r["bits"] == 4 and r["m"] == 16][0]
    out = common(args, k4m16["us"] * 1e-3 * args.steps, args.steps, k4m16["tokens_s"], "tokens/s",
                 "configs[1]: one routed SwiGLU expert (gate/up 2048->2x512, down 512->2048), K 3/4/5, m 1/4/16, "
                 "top_k 1; value = K=4 m=16", {"cases": res})
    out["cpu_baseline"] = None
    return out


# ------------------------------------------------------------------------------------------ prefill layer
def run_prefill_layer(args, torch, exl3c4):
    import exl3c4_synth as syn
    layers = build_layers(torch, 2, args.seed)             # two layers alternate (2 x 0.8 GB: no cache reuse)
    rng = np.random.default_rng(args.seed + 1)
    n_tok = 2048
    ids, w = syn.zipf_topk(rng, n_tok, E, TOP_K)
    st, off = syn.moe_scatter(ids, E)
    T = st.size
    x = torch.from_numpy(rng.standard_normal((n_tok, H)).astype(np.float16).view(np.int16)).cuda()
    stt, offt = torch.from_numpy(st).cuda(), torch.from_numpy(off).cuda()
    y = torch.zeros((T, H), dtype=torch.int16, device="cuda")
    ops = [exl3c4.make_op(exl3c4.GU_DN, BITS, CB, [L["gu_cls"]], x, stt, offt, y, n_tok, TOP_K, dn=[L["dn_cls"]])
           for L in layers]
    scratch = exl3c4.alloc_scratch(ops[0])
    steps = max(1, min(args.steps, 40))
    ms = timed_graph(torch, lambda i, s_: check_rc(exl3c4, exl3c4.launch(ops[i % 2], scratch, s_)), steps,
                     min(args.warmup, 5))
    t = ms / steps * 1e-3
    flops = 2.0 * T * (2 * W * H + H * W)
    durs = kernel_ms(torch, exl3c4, ops, scratch, exl3c4.K_GATE_UP, 10)
    gu_flops = 2.0 * T * 2 * W * H
    cnt = np.diff(off)
    live = int((cnt > 0).sum())
    out = common(args, ms, steps, n_tok / t, "tokens/s",
                 "configs[3]: routed MoE layer prefill, 2048 tokens, 512 experts at 4 bpw mul1, Zipf(1.1) "
                 "Gumbel-top-10 routing, one moe_exl3_gate_up_down launch per step (prefill path)",
                 {"rows": int(T), "live_experts": live, "max_rows_per_expert": int(cnt.max())})
    out.update({
        "mfma_frac": round(flops / t / 2.5e15, 4),
        "TFLOPs": round(flops / t / 1e12, 1),
        "packed_weight_GBps": round(live * EXPERT_BYTES / t / 1e9, 1),
        "roofline": {"bound": "mfma", "achieved": round(gu_flops / (np.mean(durs) * 1e-3) / 1e12, 1),
                     "peak": 2500.0, "unit": "TFLOP/s",
                     "frac": round(gu_flops / (np.mean(durs) * 1e-3) / 2.5e15, 4),
                     "traffic": read_traffic("k_gu_pf_prefill"),
                     "kernel": "k_gu_pf<4,mul1> (gate_up prefill GEMM)", "avg_us": round(float(np.mean(durs)) * 1e3, 1),
                     "flops_per_launch": gu_flops},
        "cpu_baseline": None,
    })
    return out


# ------------------------------------------------------------------------------------------ 48 layers
def run_stack(args, torch, exl3c4):
    """48 decode layers, all resident, K of gate_up and of down cycling through {2, 3, 4, 6, 8} (gate_up at layer l
    takes cycle[l % 5], down cycle[(l + 2) % 5]); each layer is one gate_up_down launch with down's K given apart
    (the op's dn_bits); with --stack-split, as the reference's single-K op must run it: gate_up (h_rot 1) then down
    (h_rot 1) through an h buffer. A step is 8 tokens through all the layers, each layer with its own routing draw."""
    cyc = (2, 3, 4, 6, 8)
    n_layers = args.stack_layers
    g = torch.Generator(device="cuda")
    g.manual_seed(args.seed)

    def signs(n, mag):
        s = torch.randint(0, 2, (E, n), device="cuda", generator=g).to(torch.float16) * 2 - 1
        return (s * mag).contiguous().view(torch.int16)
    draws = build_draws(torch, n_layers, args.seed + 1)
    T = M * TOP_K
    y = torch.zeros((T, H), dtype=torch.int16, device="cuda")
    h = torch.zeros((T, W), dtype=torch.int16, device="cuda")
    layer_ops, step_bytes, resident = [], 0.0, 0
    for l in range(n_layers):
        kg, kd = cyc[l % 5], cyc[(l + 2) % 5]
        gu = torch.randint(0, 256, (E, 2 * W * H * kg // 8), dtype=torch.uint8, device="cuda", generator=g)
        dn = torch.randint(0, 256, (E, H * W * kd // 8), dtype=torch.uint8, device="cuda", generator=g)
        keep = (gu, dn, signs(H, 1.0), signs(H, 1.0), signs(2 * W, 1 / np.sqrt(H)), signs(W, 1.0),
                signs(H, 1 / np.sqrt(W)))
        resident += gu.numel() + dn.numel()
        _, _, suh, suh1, svh, dsuh, dsvh = keep
        gcls = exl3c4.make_class(2 * W, H, codes=gu, suh=suh, suh1=suh1, svh=svh, dn_suh=dsuh)
        D = draws[l]
        if kg == kd or not args.stack_split:
            dcls = exl3c4.make_class(H, W, codes=dn, svh=dsvh)
            ops = [exl3c4.make_op(exl3c4.GU_DN, kg, CB, [gcls], D["x"], D["sorted_tok"], D["off"], y, M, TOP_K,
                                  dn=[dcls], dn_bits=0 if kg == kd else kd)]
        else:
            dcls = exl3c4.make_class(H, W, codes=dn, suh=dsuh, svh=dsvh)
            ops = [exl3c4.make_op(exl3c4.GATE_UP, kg, CB, [gcls], D["x"], D["sorted_tok"], D["off"], h, M, TOP_K,
                                  h_rot=1, a_rot=0),
                   exl3c4.make_op(exl3c4.DOWN, kd, CB, [dcls], h, D["sorted_tok"], D["off"], y, M, TOP_K, h_rot=1)]
        layer_ops.append((ops, keep))
        step_bytes += D["n_live"] * (2 * W * H * kg // 8 + H * W * kd // 8 + 2 * (H + H + 2 * W) + 2 * (W + H))
    scratch = torch.empty(max(exl3c4.scratch_bytes(o) for ops, _ in layer_ops for o in ops), dtype=torch.uint8,
                          device="cuda")

    # gate_up_down's counter block, zeroed once and left zeroed by every launch (exl3c4_launch_ctr: no fill dispatch a
    # layer); the layers run in order on one stream, so they share it
    ctr = torch.zeros(max([exl3c4.ctr_bytes(o) for ops, _ in layer_ops for o in ops if o.op == exl3c4.GU_DN] + [256]),
                      dtype=torch.uint8, device="cuda")

    def step(i, st):
        for ops, _ in layer_ops:
            for o in ops:
                rc = exl3c4.launch_ctr(o, scratch, ctr, st) if o.op == exl3c4.GU_DN else exl3c4.launch(o, scratch, st)
                check_rc(exl3c4, rc)
    steps = max(1, min(args.steps, 20))
    ms = timed_graph(torch, step, steps, min(args.warmup, 3))
    t = ms / steps * 1e-3
    out = common(args, ms, steps, M / t, "tokens/s",
                 f"configs[4]: {n_layers} routed MoE decode layers resident, gate_up / down K cycling "
                 "{2,3,4,6,8} per projection, 8 tokens, per-layer softmax top-10 routing; one step = all layers; "
                 + ("a layer = gate_up then down (two ops)" if args.stack_split else
                    "a layer = one gate_up_down launch (down's K apart)"),
                 {"layers": n_layers, "resident_codes_GB": round(resident / 1e9, 2),
                  "step_packed_bytes": int(step_bytes)})
    out.update({"packed_weight_GBps": round(step_bytes / t / 1e9, 1),
                "hbm_frac": round(step_bytes / t / 1e9 / HBM_PEAK_GBPS, 4), "roofline": None, "cpu_baseline": None})
    return out


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--layers", type=int, default=8)
    ap.add_argument("--draws", type=int, default=8)
    ap.add_argument("--cpu-experts", type=int, default=E,
                    help="live experts in the CPU-baseline sample (default: all of the layer's; 0: skip)")
    ap.add_argument("--seed", type=int, default=20261013)
    ap.add_argument("--config", type=int, default=3, choices=(2, 3, 4, 5),
                    help="BASELINE.json configs[n-1]: 2 one expert, 3 decode layer (default), 4 prefill layer, "
                         "5 48-layer decode stack")
    ap.add_argument("--stack-layers", type=int, default=48)
    ap.add_argument("--stack-split", action="store_true",
                    help="configs[4]: run each mixed-K layer as gate_up then down (two ops) instead of one launch")
    ap.add_argument("--no-prefill", dest="prefill", action="store_false",
                    help="with the default decode layer: skip the prefill layer's figures")
    ap.add_argument("--op-only", action="store_true",
                    help="the decode layer's op graph alone (gate_up_down launches back to back), for a profiler")
    ap.add_argument("--no-stack", dest="stack", action="store_false",
                    help="with the default decode layer: skip the 48-layer stack's figures")
    ap.add_argument("--no-peaks", dest="peaks", action="store_false",
                    help="skip the measured HBM and GEMM ceilings (peaks_measured, roofline frac_measured)")
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
    run = {2: run_single_expert, 3: run_decode_layer, 4: run_prefill_layer, 5: run_stack}[args.config]
    out = run(args, torch, exl3c4)
    if out.get("op_only"):
        print(json.dumps(out), flush=True)
        return
    peaks = measured_peaks(torch) if args.peaks else None
    if args.config == 3 and args.prefill:
        # the prefill layer measured in the same run, its figures beside the decode line's
        torch.cuda.empty_cache()
        pf = run_prefill_layer(args, torch, exl3c4)
        out["prefill"] = {"workload": pf["config"]["workload"], "rows": pf["config"]["rows"],
                          "max_rows_per_expert": pf["config"]["max_rows_per_expert"],
                          "us_per_layer": round(pf["ms_per_step"] * 1e3, 1), "tokens_per_s": pf["value"],
                          "TFLOPs": pf["TFLOPs"], "mfma_frac": pf["mfma_frac"], "roofline": pf["roofline"]}
    if args.config == 3 and args.stack:
        # the 48-layer stack measured in the same run
        torch.cuda.empty_cache()
        sk = run_stack(args, torch, exl3c4)
        out["stack"] = {"workload": sk["config"]["workload"], "layers": sk["config"]["layers"],
                        "resident_codes_GB": sk["config"]["resident_codes_GB"],
                        "us_per_step": round(sk["ms_per_step"] * 1e3, 1), "tokens_per_s": sk["value"],
                        "packed_weight_GBps": sk["packed_weight_GBps"], "hbm_frac": sk["hbm_frac"]}
        torch.cuda.empty_cache()
    if peaks:
        out["peaks_measured"] = peaks
        hbm = max(peaks["hbm_read_GBps"], peaks["hbm_copy_GBps"])
        mf = max(peaks["mfma_f16_TFLOPs"], peaks["fp16_gemm_TFLOPs"])
        rf = out.get("roofline")
        if rf is not None:
            add_measured(rf, hbm if rf["unit"] == "GB/s" else mf)
        rv = out.get("roofline_valu")
        if rv is not None:
            rv["peak_measured"] = peaks["valu_Ginstr_s"]
            rv["frac_measured"] = round(rv["achieved"] / peaks["valu_Ginstr_s"], 4)
        if "prefill" in out:
            add_measured(out["prefill"]["roofline"], mf)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
