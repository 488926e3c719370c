"""RngdKVConnector on the host path: construction, metadata, and a prefill and a
decode process handing KV over /dev/shm (the reference's
tests/test_connector_tcp.py shape, over the shm transport)."""
import multiprocessing as mp
import os
import tempfile

import numpy as np

from rngd_pd_amd.connector import transport as kv
from rngd_pd_amd.connector.kv_base import KVConnectorBase_V1
from rngd_pd_amd.connector.rngd_kv import (KVConnectorRole, RngdKVConnector,
                                           RngdKVConnectorMetadata)

NL, NKV, S, HD = 6, 8, 16, 128
SEED = 1234


def _ref():
    rng = np.random.default_rng(SEED)
    ck = [rng.standard_normal((NKV, S, HD)).astype(np.float32) for _ in range(NL)]
    cv = [rng.standard_normal((NKV, S, HD)).astype(np.float32) for _ in range(NL)]
    return ck, cv


def _prefill_proc(root, wire):
    kv.WIRE = wire
    conn = RngdKVConnector(KVConnectorRole.WORKER, req_id="reqT", transport=kv.ShmTransport(root),
                           n_layers=NL)
    ck, cv = _ref()
    for i in range(NL):
        conn.save_kv_layer(f"layer.{i}", (ck[i], cv[i]))
    conn.wait_for_save()


def _decode_proc(root, out_path):
    dk = [np.zeros((NKV, S, HD), np.float32) for _ in range(NL)]
    dv = [np.zeros((NKV, S, HD), np.float32) for _ in range(NL)]
    conn = RngdKVConnector(KVConnectorRole.WORKER, req_id="reqT", transport=kv.ShmTransport(root),
                           n_layers=NL)
    conn.register_kv_caches((dk, dv))
    conn.bind_connector_metadata(conn.build_connector_meta(None))
    conn.start_load_kv()
    for i in range(NL):
        conn.wait_for_layer_load(f"layer.{i}")       # blocks until prefill has pushed it
    np.savez(out_path, **{f"k{i}": dk[i] for i in range(NL)}, **{f"v{i}": dv[i] for i in range(NL)})


def test_two_processes_over_shm():
    """Decode starts first and blocks; prefill pushes; fp16 wire loss < 1e-6 and
    bf16 wire bit-exact for bf16 truncation."""
    ctx = mp.get_context("spawn")
    for wire in ("fp16", "bf16"):
        with tempfile.TemporaryDirectory(dir="/dev/shm" if os.access("/dev/shm", os.W_OK) else None) as root:
            out = os.path.join(root, "decoded.npz")
            dp = ctx.Process(target=_decode_proc, args=(root, out))
            dp.start()
            pp = ctx.Process(target=_prefill_proc, args=(root, wire))
            pp.start()
            pp.join(120)
            dp.join(120)
            assert pp.exitcode == 0 and dp.exitcode == 0
            z = np.load(out)
            ck, cv = _ref()
            for i in range(NL):
                for got, a in ((z[f"k{i}"], ck[i]), (z[f"v{i}"], cv[i])):
                    if wire == "fp16":
                        assert np.abs(got - a.astype(np.float16).astype(np.float32)).max() < 1e-6
                    else:
                        np.testing.assert_array_equal(got.view(np.uint32),
                                                      a.view(np.uint32) >> 16 << 16)


def test_construction_and_metadata():
    tr = kv.InProcTransport()
    c = RngdKVConnector(KVConnectorRole.WORKER, "req9", tr, 4)
    assert isinstance(c, KVConnectorBase_V1)
    assert (c.req_id, c.t, c.n_layers, c.role) == ("req9", tr, 4, KVConnectorRole.WORKER)
    meta = c.build_connector_meta(None)
    assert isinstance(meta, RngdKVConnectorMetadata)
    assert meta.load_layers == meta.save_layers == [f"layer.{i}" for i in range(4)]
    sched = RngdKVConnector(KVConnectorRole.SCHEDULER, req_id="r", n_layers=2)
    assert sched.build_connector_meta(None).save_layers == []

    class Req:
        kv_ready_tokens = 40
    assert c.get_num_new_matched_tokens(Req(), 10) == (30, True)
    assert c.get_num_new_matched_tokens(Req(), 40) == (None, False)
    assert c.get_finished(set()) == (None, None)


def test_vllm_style_construction_reads_extra_config():
    class Xfer:
        kv_connector_extra_config = {"req_id": "fromcfg", "n_layers": 3, "frame_tokens": 64}

    class Cfg:
        kv_transfer_config = Xfer()
    c = RngdKVConnector(Cfg(), KVConnectorRole.WORKER, None, transport=kv.InProcTransport())
    assert (c.req_id, c.n_layers, c.frame_tokens) == ("fromcfg", 3, 64)


def test_dict_caches_and_stacked_layer():
    tr = kv.InProcTransport()
    old = kv.WIRE
    kv.WIRE = "bf16"
    try:
        pf = RngdKVConnector(KVConnectorRole.WORKER, req_id="d", transport=tr, n_layers=2)
        rng = np.random.default_rng(0)
        layers = [rng.standard_normal((2, NKV, S, HD)).astype(np.float32) for _ in range(2)]
        for i, a in enumerate(layers):
            pf.save_kv_layer(f"model.layers.{i}", a)          # stacked [2, ...] form
        caches = {f"model.layers.{i}": (np.zeros((NKV, S, HD), np.float32),
                                        np.zeros((NKV, S, HD), np.float32)) for i in range(2)}
        dc = RngdKVConnector(KVConnectorRole.WORKER, req_id="d", transport=tr)
        dc.register_kv_caches(caches)
        assert dc.n_layers == 2
        dc.start_load_kv()
        for i in range(2):
            k, v = dc.wait_for_layer_load(f"model.layers.{i}")
            want = (layers[i].view(np.uint32) >> 16 << 16).view(np.float32)
            np.testing.assert_array_equal(caches[f"model.layers.{i}"][0], want[0])
            np.testing.assert_array_equal(v, want[1])
    finally:
        kv.WIRE = old


def test_load_request_consumes_only_its_own_files():
    """The decode worker's host-path load (serving/cluster.py:438-467): zeroed f32
    K [L, Hkv, D, S] / V [L, Hkv, S, D], every layer loaded, then the request's
    files gone; another request whose id shares a prefix keeps its files."""
    from rngd_pd_amd.connector.rngd_kv import load_request
    rng = np.random.default_rng(SEED)
    K = rng.standard_normal((NL, NKV, HD, S)).astype(np.float32)
    V = rng.standard_normal((NL, NKV, S, HD)).astype(np.float32)
    with tempfile.TemporaryDirectory(dir="/dev/shm" if os.access("/dev/shm", os.W_OK) else None) as root:
        t = kv.ShmTransport(root)
        for req in ("r7", "r77"):
            conn = RngdKVConnector(KVConnectorRole.WORKER, req_id=req, transport=t, n_layers=NL)
            for i in range(NL):
                conn.save_kv_layer(f"layer.{i}", (K[i], V[i]))
        old = kv.WIRE
        try:
            kv.WIRE = "bf16"
            for i in range(NL):                       # r7 goes over the bf16 wire
                for which, arr in (("k", K[i]), ("v", V[i])):
                    t.push(f"r7/layer.{i}/{which}", kv.ser(arr))
        finally:
            kv.WIRE = old
        gotK, gotV, ms = load_request("r7", NL, NKV, HD, S, transport=t)
        trunc = lambda a: (a.view(np.uint32) >> 16 << 16).view(np.float32)   # noqa: E731
        np.testing.assert_array_equal(gotK, trunc(K))
        np.testing.assert_array_equal(gotV, trunc(V))
        assert ms >= 0
        left = sorted(os.listdir(root))
        assert left == sorted(f"r77__layer.{i}__{w}" for i in range(NL) for w in "kv")
