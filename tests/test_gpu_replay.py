"""Replay across processes (the reference's R8, tests/gpu/test_exl3r4d.py:20-22: the same case three times in three
processes, byte-identical): gate_up_down's output bytes on the replay cases (tests/replay_child.py) in this process
and in three child processes started one after another, all equal. Within one process the parity tests replay
already; across processes the scratch, the counter blocks and the allocator's addresses start afresh."""
import os
import subprocess
import sys

import pytest

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))


@pytest.fixture(scope="module")
def torch_cuda():
    torch = pytest.importorskip("torch")
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import exl3c4
    exl3c4.lib()
    return torch


def test_replay_in_three_processes_is_byte_identical(torch_cuda):
    import replay_child
    here = replay_child.replay()
    print(f"in process: {here}", flush=True)
    for run in range(3):
        print(f"child process {run + 1} of 3", flush=True)
        r = subprocess.run([sys.executable, "-u", os.path.join(HERE, "replay_child.py")], capture_output=True,
                           text=True, timeout=100)
        assert r.returncode == 0, f"child {run + 1} exited {r.returncode}: {r.stdout[-2000:]} {r.stderr[-2000:]}"
        got = dict(line.split()[1:3] for line in r.stdout.splitlines() if line.startswith("sha "))
        assert got == here, f"child {run + 1}: {got} != {here}"
