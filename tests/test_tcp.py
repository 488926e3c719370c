"""The native cross-node tcp transport (librngdpd_net.so) on the CPU.

Behaviours of the reference's relay, client and adapter tests
(tests/test_kv_tcp.py, tests/test_connector_tcp.py), wire interop with a
Python restatement of the reference's protocol (oracle/tcpkv.py) in both
directions, and the CRC-32 against zlib.
"""
import multiprocessing as mp
import os
import socket
import struct
import threading
import time
import zlib

import numpy as np
import pytest

from oracle import tcpkv as otcp
from rngd_pd_amd import airm, rm_compat  # noqa: F401
from tests.rm_doubles import check_kv_transport
from rngd_pd_amd.connector import tcp
from rngd_pd_amd.connector import transport as kv


@pytest.fixture()
def relay():
    srv = tcp.TcpKVServer(0, "127.0.0.1").start()
    port = srv.wait_ready()
    c = tcp.TcpKVClient("127.0.0.1", port)
    yield srv, port, c
    c.close()
    srv.stop()


def test_crc32_matches_zlib():
    assert tcp.crc32(b"123456789") == 0xCBF43926            # the CRC-32 check value
    rng = np.random.default_rng(0)
    for n in (0, 1, 15, 16, 17, 255, 4096 + 3, 1 << 20):
        data = rng.bytes(n)
        assert tcp.crc32(data) == zlib.crc32(data), n
        assert tcp.crc32(data[n // 3:], tcp.crc32(data[:n // 3])) == zlib.crc32(data)


def test_round_trip_is_byte_exact_and_consumed(relay):
    _srv, _port, c = relay
    blob = np.random.default_rng(0).bytes(3 << 20)
    c.push("r/layer.0/k", blob)
    assert bytes(c.take("r/layer.0/k", timeout=1)) == blob
    with pytest.raises(TimeoutError):
        c.take("r/layer.0/k", timeout=0.05)                  # handed out once


def test_take_waits_for_a_later_push(relay):
    _srv, port, c = relay
    got = {}
    t = threading.Thread(target=lambda: got.update(v=bytes(c.take("late", timeout=5))))
    t.start()
    time.sleep(0.2)
    other = tcp.TcpKVClient("127.0.0.1", port)
    other.push("late", b"xyz")
    t.join(5)
    other.close()
    assert got.get("v") == b"xyz"


def test_connections_are_reused(relay):
    _srv, _port, c = relay
    for i in range(20):
        c.push(f"k{i}", b"a" * 1000)
        c.take(f"k{i}")
    assert c.idle_connections() == 1


def test_concurrent_clients(relay):
    _srv, _port, c = relay
    blobs = {f"q{i}/layer.{j}/k": os.urandom(50_000) for i in range(8) for j in range(4)}
    errs = []

    def worker(keys):
        try:
            for k in keys:
                c.push(k, blobs[k])
            for k in keys:
                if bytes(c.take(k, timeout=5)) != blobs[k]:
                    errs.append(k)
        except Exception as e:                               # noqa: BLE001 - reported below
            errs.append(repr(e))
    keys = sorted(blobs)
    ts = [threading.Thread(target=worker, args=(keys[i::8],)) for i in range(8)]
    [t.start() for t in ts]
    [t.join(30) for t in ts]
    assert errs == []
    st = c.stats()
    assert (st["pushed"], st["taken"], st["keys"], st["crc_errors"]) == (32, 32, 0, 0)


def test_corrupt_push_is_rejected(relay):
    _srv, port, c = relay
    s = socket.create_connection(("127.0.0.1", port))
    data = b"payload"
    s.sendall(b"P" + struct.pack("<i", 1) + b"k" + struct.pack("<qI", len(data), 12345) + data)
    assert s.recv(2) == b"ER"
    s.close()
    assert c.stats()["crc_errors"] == 1
    with pytest.raises(TimeoutError):
        c.take("k", timeout=0.05)


def test_expired_blobs_are_dropped(relay):
    srv, _port, c = relay
    srv.ttl_s = 0.0
    c.push("old", b"x")
    time.sleep(1.2)                                          # expiry runs every 0.5 s
    assert c.stats()["expired"] == 1 and srv.stats["expired"] == 1


def test_oversize_take_keeps_the_blob(relay):
    _srv, _port, c = relay
    blob = os.urandom(5000)
    c.push("big", blob)
    small = bytearray(100)
    with pytest.raises(tcp.BlobTooLarge) as e:
        c.take_into("big", small, timeout=1)
    assert e.value.size == 5000
    out = bytearray(8192)
    assert c.take_into("big", out, timeout=1) == 5000 and bytes(out[:5000]) == blob


def test_parse_addr():
    assert tcp.parse_addr("relay.ns.svc:6000") == ("relay.ns.svc", 6000)
    assert tcp.parse_addr("relay") == ("relay", 5577)


def test_interop_native_client_with_reference_protocol_relay():
    r = otcp.Relay()
    r.start()
    try:
        c = tcp.TcpKVClient("127.0.0.1", r.port)
        blob = np.random.default_rng(3).bytes(1 << 20)
        c.push("req/layer.3/v", blob)
        assert r.store["req/layer.3/v"] == (blob, zlib.crc32(blob))
        assert bytes(c.take("req/layer.3/v", timeout=1)) == blob
        with pytest.raises(TimeoutError):
            c.take("missing", timeout=0.05)
        assert otcp.push(r.port, "bad", b"zz", crc=7) == b"ER"
        c.close()
    finally:
        r.stop()


def test_interop_reference_protocol_client_with_native_relay(relay):
    _srv, port, c = relay
    blob = np.random.default_rng(4).bytes(70_000)
    assert otcp.push(port, "a/b", blob) == b"OK"
    data, crc = otcp.take(port, "a/b")
    assert data == blob and crc == zlib.crc32(blob)
    assert otcp.take(port, "a/b", wait_ms=50) == (None, 0)
    c.push("from-native", blob[:10])
    assert otcp.take(port, "from-native")[0] == blob[:10]
    assert otcp.push(port, "zero-crc", b"unchecked", crc=0) == b"OK"   # crc 0 = unchecked


@pytest.fixture()
def tcp_env(monkeypatch):
    srv = tcp.TcpKVServer(0, "127.0.0.1").start()
    monkeypatch.setenv("AIRM_KV_TCP_ADDR", f"127.0.0.1:{srv.wait_ready()}")
    monkeypatch.delenv("AIRM_KV_TRANSPORT", raising=False)
    kv.reset_selection()
    yield srv
    for t in kv._SELECTOR.held().values():
        t.close()
    kv.reset_selection()
    srv.stop()


def test_tcp_by_name_is_one_shared_instance(tcp_env, monkeypatch):
    monkeypatch.setenv("AIRM_KV_TRANSPORT", "tcp")
    a, b = kv.select_transport(), kv.select_transport()
    assert isinstance(a, airm.TcpTransport) and a is b
    assert a.remote == ("127.0.0.1", tcp_env.port)
    assert a.handshake_metadata() == {"tcp": f"127.0.0.1:{tcp_env.port}"}


def test_needs_an_address(monkeypatch):
    monkeypatch.delenv("AIRM_KV_TCP_ADDR", raising=False)
    t = tcp.TcpTransport()
    with pytest.raises(ValueError):
        t.push("k", b"x")


def test_adapter_conformance_and_payload(tcp_env, monkeypatch):
    monkeypatch.delenv("AIRM_KV_TCP_ADDR")
    t = airm.TcpTransport()                                  # conformance starts its own relay
    check_kv_transport(t)
    assert t.measurements[-1].tags["kv_transport"] == "tcp"
    t.close()
    monkeypatch.setenv("AIRM_KV_TCP_ADDR", f"127.0.0.1:{tcp_env.port}")
    t = airm.TcpTransport()
    src, dst, layout = t.conformance_case()
    kv_in = np.random.default_rng(1).standard_normal((2, 2, 4, 2, 8)).astype(np.float32)
    plan = t.plan("q", src, dst, layout, layout, (0, 4))
    assert plan.detail["server"] == f"127.0.0.1:{tcp_env.port}"
    res = t.wait(t.submit(plan, kv=kv_in), timeout_s=5)
    assert res.ok
    got = t.take(plan).reshape(kv_in.shape)
    np.testing.assert_array_equal(got.view(np.uint32), kv_in.view(np.uint32) >> 16 << 16)
    t.close()


NL, NKV, S, HD, SEED = 6, 8, 16, 128, 1234


def _ref_kv():
    rng = np.random.default_rng(SEED)
    ck = [rng.standard_normal((NKV, S, HD)).astype(np.float32) for _ in range(NL)]
    cv = [rng.standard_normal((NKV, S, HD)).astype(np.float32) for _ in range(NL)]
    return ck, cv


def _prefill_proc(port):
    from rngd_pd_amd.connector.rngd_kv import KVConnectorRole, RngdKVConnector
    tr = tcp.TcpTransport(remote=("127.0.0.1", port))
    conn = RngdKVConnector(KVConnectorRole.WORKER, req_id="reqT", transport=tr, n_layers=NL)
    ck, cv = _ref_kv()
    for i in range(NL):
        conn.save_kv_layer(f"layer.{i}", (ck[i], cv[i]))
    conn.wait_for_save()
    tr.close()


def _decode_proc(port, out_path):
    from rngd_pd_amd.connector.rngd_kv import KVConnectorRole, RngdKVConnector
    tr = tcp.TcpTransport(remote=("127.0.0.1", port))
    dk = [np.zeros((NKV, S, HD), np.float32) for _ in range(NL)]
    dv = [np.zeros((NKV, S, HD), np.float32) for _ in range(NL)]
    conn = RngdKVConnector(KVConnectorRole.WORKER, req_id="reqT", transport=tr, n_layers=NL)
    conn.register_kv_caches((dk, dv))
    conn.bind_connector_metadata(conn.build_connector_meta(None))
    conn.start_load_kv()
    for i in range(NL):
        conn.wait_for_layer_load(f"layer.{i}")
    np.savez(out_path, **{f"k{i}": dk[i] for i in range(NL)}, **{f"v{i}": dv[i] for i in range(NL)})
    tr.close()


def test_connector_across_processes_fp16_wire(tmp_path):
    """tests/test_connector_tcp.py: prefill and decode in separate processes,
    6 layers of seed-1234 KV over the relay; equal to the fp16 round trip."""
    srv = tcp.TcpKVServer(0, "127.0.0.1").start()
    port = srv.wait_ready()
    out = str(tmp_path / "decode.npz")
    ctx = mp.get_context("spawn")
    dp = ctx.Process(target=_decode_proc, args=(port, out))
    dp.start()                                               # decode first: it blocks pulling
    pp = ctx.Process(target=_prefill_proc, args=(port,))
    pp.start()
    pp.join(120)
    dp.join(120)
    srv.stop()
    assert pp.exitcode == 0 and dp.exitcode == 0
    ck, cv = _ref_kv()
    z = np.load(out)
    ref16 = lambda a: a.astype(np.float16).astype(np.float32)   # noqa: E731
    for i in range(NL):
        np.testing.assert_array_equal(z[f"k{i}"], ref16(ck[i]))
        np.testing.assert_array_equal(z[f"v{i}"], ref16(cv[i]))
