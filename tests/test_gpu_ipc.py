"""Same-GPU IPC handoff between a prefill process and a decode process.

Two child processes share the GPU: the producer saves requests through the
connector on the ipc transport (frames stay in its HBM, exported through one
IPC handle; 2 slots for 4 requests, so slots must come back), the consumer
scatters them from the producer's memory into its paged cache and checks them
bit for bit against a local pack + scatter of the same KV (tests/ipc_peer.py).
"""
import os
import subprocess
import sys

import pytest

pytestmark = pytest.mark.gpu

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_ipc_two_process_handoff(tmp_path):
    n = 4
    env = dict(os.environ, PD_KV_PULL_TIMEOUT="60", PYTHONPATH=REPO)
    peer = os.path.join(REPO, "tests", "ipc_peer.py")
    root = str(tmp_path / "ipc")
    print(f"ipc handoff: {n} requests under {root}", flush=True)
    procs = [subprocess.Popen([sys.executable, "-u", peer, role, root, str(n)], env=env,
                              stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
             for role in ("producer", "consumer")]
    outs = []
    try:
        for p in procs:
            outs.append(p.communicate(timeout=100)[0])
    finally:
        for p in procs:
            if p.poll() is None:
                p.kill()
                p.wait()
    log = "\n".join(f"--- {r}\n{o}" for r, o in zip(("producer", "consumer"), outs))
    assert procs[0].returncode == 0 and procs[1].returncode == 0, log
    assert f"ipc consumer ok {n}" in outs[1], log
    assert outs[1].count("bit-exact") == n, log
    assert not os.listdir(root), f"files left behind: {os.listdir(root)}"
