"""One side of the two-process same-GPU IPC handoff test (run as a script).

    python tests/ipc_peer.py producer ROOT N
    python tests/ipc_peer.py consumer ROOT N

The producer saves N requests through RngdKVConnector on the ipc transport,
with 2 frame slots, so slots must come back from the consumer. The consumer
loads them into a paged cache through the connector and checks each against a
local pack + scatter of the same seeded KV, bit for bit. Both print one line
per step and exit non-zero on any mismatch.
"""
import os
import sys

sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.abspath(__file__))))

L, H, D, S = 4, 8, 128, 512
LENGTHS = [509, 64, 300, 512]


def kv_of(torch, r, dev):
    gen = torch.Generator(device=dev).manual_seed(100 + r)
    return torch.randn((L, 2, S, H, D), generator=gen, device=dev).to(torch.bfloat16)


def producer(root, n):
    import torch
    from rngd_pd_amd.connector.ipc import IpcTransport
    from rngd_pd_amd.connector.rngd_kv import KVConnectorRole, RngdKVConnector
    dev = torch.device("cuda:0")
    t = IpcTransport(root, n_slots=2)
    for r in range(n):
        kv = kv_of(torch, r, dev)
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
    from rngd_pd_amd.connector import ipc
    from rngd_pd_amd.connector.ipc import IpcTransport
    from rngd_pd_amd.connector.rngd_kv import KVConnectorRole, RngdKVConnector
    from rngd_pd_amd.engines.paged_cache import PagedKVCache
    from rngd_pd_amd.kernels import handoff as K
    dev = torch.device("cuda:0")
    t = IpcTransport(root)
    cache = PagedKVCache(L, n * (S // 16) + 4, H, D, device=dev, seed=7)
    want = PagedKVCache(L, n * (S // 16) + 4, H, D, device=dev, seed=7)
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
        # The same KV packed and scattered locally, into the same block ids.
        kv = kv_of(torch, r, dev)
        frame = K.pack_kv(kv[:, 0], kv[:, 1], P, S)
        want.allocate(req, P)
        assert want.blocks(req) == cache.blocks(req)
        K.scatter_paged(frame, want.table(req), P, S, want.k, want.v)
        back = cache.read_frame(req, P, S)
        torch.cuda.synchronize()
        ok = (torch.equal(cache.k.view(torch.int16), want.k.view(torch.int16))
              and torch.equal(cache.v.view(torch.int16), want.v.view(torch.int16))
              and torch.equal(back.view(torch.int16), frame.view(torch.int16)))
        bad += not ok
        print(f"consumer req{r} P={P}: {'bit-exact' if ok else 'MISMATCH'}", flush=True)
    ipc.close_opened()
    print(f"ipc consumer {'ok' if bad == 0 else 'FAILED'} {n}", flush=True)
    return 1 if bad else 0


if __name__ == "__main__":
    role, root, n = sys.argv[1], sys.argv[2], int(sys.argv[3])
    sys.exit(producer(root, n) or 0 if role == "producer" else consumer(root, n))
