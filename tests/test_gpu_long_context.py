"""The long-context layer-pipelined save, against the oracle.

16 requests of 2048 tokens of Llama-3.1-8B KV (32 layers, 8 KV heads, head_dim
128, bf16; 4 GiB on the wire) go through RngdKVConnector.save_kv_layer with
frame_tokens=2048, one layer at a time, while the prefill's stream runs a
[32768, 4096] x [4096, 4096] bf16 GEMM per layer (the reference's frame producer
hands each layer group to its writer while the next group computes,
engines/prefill_full.py:366-384). The device save packs on its side stream
after waiting for the prefill stream, so each layer's save overlaps the next
layer's GEMM. Every published file must equal, byte for byte, the oracle's
ser() of the oracle's frame for that layer; the GEMM's result must be intact.
"""
import os
import shutil
import tempfile

import numpy as np
import pytest
import torch

from oracle import native as orc
from oracle import wire as owire
from tests._util import to_host

pytestmark = pytest.mark.gpu

L, H, D = 32, 8, 128


def _widen(u16):
    return (u16.astype(np.uint32) << 16).view(np.float32)


def test_long_context_save_matches_oracle(cuda):
    from rngd_pd_amd.connector.rngd_kv import KVConnectorRole, RngdKVConnector
    from rngd_pd_amd.connector.transport import ShmTransport
    n_req, T, hidden = 16, 2048, 4096
    gen = torch.Generator(device=cuda).manual_seed(4)
    kv = [torch.randn((L, 2, T, H, D), generator=gen, device=cuda).to(torch.bfloat16)
          for _ in range(n_req)]
    x = torch.randn((n_req * T, hidden), generator=gen, device=cuda).to(torch.bfloat16)
    w = torch.randn((hidden, hidden), generator=gen, device=cuda).to(torch.bfloat16) / 64
    y = torch.empty((n_req * T, hidden), dtype=torch.bfloat16, device=cuda)
    root = tempfile.mkdtemp(prefix="pdk_long_", dir="/dev/shm" if os.path.isdir("/dev/shm") else None)
    try:
        t = ShmTransport(root)
        conns = [RngdKVConnector(KVConnectorRole.WORKER, req_id=f"lc{i}", transport=t,
                                 n_layers=L, frame_tokens=T) for i in range(n_req)]
        print(f"long context: {n_req} x {T} tokens, {L} layers, GEMM per layer", flush=True)
        for li in range(L):
            torch.matmul(x, w, out=y)
            for i, c in enumerate(conns):
                c.save_kv_layer(f"layer.{li}", (kv[i][li, 0], kv[i][li, 1]), num_tokens=T)
        for c in conns:
            c.wait_for_save()
        torch.cuda.synchronize()
        want_y = (x[:256].float() @ w.float())
        torch.testing.assert_close(y[:256].float(), want_y, atol=0.05, rtol=0.02)
        assert len(os.listdir(root)) == n_req * L * 2
        for i, c in enumerate(conns):
            c.close()
            bits = to_host(kv[i])                                  # [L, 2, T, H, D]
            frame = orc.pack_kv(bits[:, 0], bits[:, 1], T, T)      # [L, 2, H*D*T]
            for li in range(L):
                for which, part, shape in (("k", 0, (H, D, T)), ("v", 1, (H, T, D))):
                    want = owire.ser(_widen(frame[li, part]).reshape(shape), "bf16")
                    with open(os.path.join(root, f"lc{i}__layer.{li}__{which}"), "rb") as f:
                        got = f.read()
                    assert got == want, f"request {i} layer {li} {which}"
            print(f"request {i}: 64 files equal the oracle's", flush=True)
    finally:
        shutil.rmtree(root, ignore_errors=True)
