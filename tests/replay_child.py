"""One replay of the replay cases in a process of its own: prints `sha <case> <sha256 of the output bytes>` a case.

Run by tests/test_gpu_replay.py as a child process (never imported by pytest's collection: no test_ prefix). The
cases are built from fixed seeds, so every process builds the same inputs; the hashes say whether a launch's output
depends on anything a process leaves behind (scratch contents, counter blocks, the allocator's addresses).
"""
import hashlib
import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for sub in ("", "oracle", "radiance-exl3_amd", "tests"):
    p = os.path.join(ROOT, sub)
    if p not in sys.path:
        sys.path.insert(0, p)

# name -> Case arguments: gate_up_down as one kernel (k_gd: 40 rows of 8-row runs), the decode pair below the
# one-kernel threshold (k_gu -> k_gepi -> k_dn), and the prefill path (a plan, runs cut into several chunks, drops)
CASES = {
    "one_kernel": dict(seed=61, n_tok=8, top_k=5, n_expert=16, geoms=[(512, 256)], bits=4, cb="mul1"),
    "decode_pair": dict(seed=62, n_tok=3, top_k=4, n_expert=8, geoms=[(256, 256), (384, 128)], bits=3, cb="mcg"),
    "prefill": dict(seed=40, n_tok=200, top_k=2, n_expert=4, geoms=[(256, 256), (384, 128)], bits=4, cb="mul1",
                    drop=0.1, protect_tail=2, routing="zipf"),
}


def replay():
    """{case name: sha256 hex of gate_up_down's output bytes}, one launch a case on cuda:0."""
    from cases import Case, Dev
    out = {}
    for name, kw in CASES.items():
        dev = Dev(Case(**kw))
        y = dev.gate_up_down()
        assert dev.status in (None, 0), f"{name}: status word {dev.status}"   # None: no single kernel ran
        out[name] = hashlib.sha256(y.tobytes()).hexdigest()
    return out


if __name__ == "__main__":
    for name, h in replay().items():
        print(f"sha {name} {h}", flush=True)
