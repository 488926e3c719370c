"""One side of the two-process same-GPU IPC handoff test (run as a script).

    python tests/ipc_peer.py producer ROOT N
    python tests/ipc_peer.py consumer ROOT N

The producer saves N requests through RngdKVConnector on the ipc transport,
with 2 frame slots, so slots must come back from the consumer. Request r's KV
is random bf16 bit patterns from numpy seed 100 + r, which both sides draw.
The consumer loads every request into a paged cache through the connector and
checks the whole cache, bit for bit, against the oracle's pack + scatter of
the same bits into the same block ids, and each request's frame read back from
the cache against the oracle's S-wide frame. Both print one line per step and
exit non-zero on any mismatch.
"""
import os
import sys

sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.abspath(__file__))))

import numpy as np  # noqa: E402

L, H, D, S = 4, 8, 128, 512
LENGTHS = [509, 64, 300, 512]


def kv_bits(r):
    """Request r's prefill KV [L, 2, S, H, D] as bf16 bit patterns."""
    return np.random.default_rng(100 + r).integers(0, 1 << 16, (L, 2, S, H, D), dtype=np.uint16)


def producer(root, n):
    import torch
    from rngd_pd_amd.connector.ipc import IpcTransport
    from rngd_pd_amd.connector.rngd_kv import KVConnectorRole, RngdKVConnector
    from tests._util import to_dev
    dev = torch.device("cuda:0")
    t = IpcTransport(root, n_slots=2)
    for r in range(n):
        kv = to_dev(kv_bits(r), dev)
        c = RngdKVConnector(KVConnectorRole.WORKER, req_id=f"req{r}", transport=t, n_layers=L,
                            frame_tokens=S)
        for layer in range(L):
            c.save_kv_layer(f"layer.{layer}", (kv[layer, 0], kv[layer, 1]),
                            num_tokens=LENGTHS[r % len(LENGTHS)])
        c.wait_for_save()
        c.close()
        print(f"producer published req{r}", flush=True)
    t.close()                                     # waits for the consumer's releases
    print("producer done", flush=True)


def consumer(root, n):
    import torch
    from oracle import native as orc
    from rngd_pd_amd.connector import ipc
    from rngd_pd_amd.connector.ipc import IpcTransport
    from rngd_pd_amd.connector.rngd_kv import KVConnectorRole, RngdKVConnector
    from rngd_pd_amd.engines.paged_cache import PagedKVCache
    from tests._util import to_host
    dev = torch.device("cuda:0")
    t = IpcTransport(root)
    nb = n * (S // 16) + 4
    cache = PagedKVCache(L, nb, H, D, device=dev, seed=7)
    want_k = np.zeros((L, nb, H, 16, D), np.uint16)      # the cache starts zeroed
    want_v = np.zeros((L, nb, H, D, 16), np.uint16)
    bad = 0
    for r in range(n):
        P = LENGTHS[r % len(LENGTHS)]
        req = f"req{r}"
        c = RngdKVConnector(KVConnectorRole.WORKER, req_id=req, transport=t, n_layers=L)
        c.register_kv_caches(cache.view(req, num_tokens=P, S=S))
        c.bind_connector_metadata(c.build_connector_meta(None))
        c.start_load_kv()
        for layer in range(L):
            c.wait_for_layer_load(f"layer.{layer}")
        c.close()
        kv = kv_bits(r)
        frame = orc.pack_kv(kv[:, 0], kv[:, 1], P, S)
        orc.scatter_paged(frame, np.asarray(cache.blocks(req), np.int32), P, S, H, D,
                          want_k, want_v)
        back = cache.read_frame(req, P, S)
        torch.cuda.synchronize()
        ok = (np.array_equal(to_host(cache.k), want_k) and np.array_equal(to_host(cache.v), want_v)
              and np.array_equal(to_host(back), frame))
        bad += not ok
        print(f"consumer req{r} P={P}: {'bit-exact vs oracle' if ok else 'MISMATCH'}", flush=True)
    ipc.close_opened()
    print(f"ipc consumer {'ok' if bad == 0 else 'FAILED'} {n}", flush=True)
    return 1 if bad else 0


if __name__ == "__main__":
    role, root, n = sys.argv[1], sys.argv[2], int(sys.argv[3])
    sys.exit(producer(root, n) or 0 if role == "producer" else consumer(root, n))
