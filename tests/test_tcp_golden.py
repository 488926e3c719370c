"""The tcp KV wire against bytes the reference's own relay and client produced.

tests/golden/tcp_wire.json was recorded from the reference's connector/tcpkv.py
(TcpKVServer and TcpKVClient over loopback, wire at :9-17) by
tests/golden/make_tcp_golden.py: a scripted session of pushes, takes (present,
absent, empty, unchecked), a push with a wrong CRC and stats, each as the
bytes the client sent and the bytes the relay answered. Replayed here:

* to the native relay (librngdpd_net.so) and to the oracle's restatement of
  the relay: every answer, stats JSON included, must be the reference's
  byte for byte;
* from the native client, against a scripted peer that answers with the
  reference relay's bytes: every request must be the reference client's
  byte for byte, and every call must return what the reference client did.
"""
import json
import os
import socket
import struct
import threading
import zlib

import numpy as np
import pytest

from oracle import tcpkv as otcp
from rngd_pd_amd.connector import tcp

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "tcp_wire.json")


@pytest.fixture(scope="module")
def session():
    with open(GOLDEN) as f:
        fx = json.load(f)
    rng = np.random.default_rng(fx["blobs"]["seed"])
    blobs = {"k": rng.bytes(fx["blobs"]["k"]), "v": rng.bytes(fx["blobs"]["v"]), "empty": b""}
    for e in fx["exchanges"]:
        e["client"], e["server"] = bytes.fromhex(e["client"]), bytes.fromhex(e["server"])
        if "blob" in e:
            e["data"] = blobs[e["blob"]][:e.get("length")]
    return fx["exchanges"]


def _recv(s, n):
    out = b""
    while len(out) < n:
        chunk = s.recv(n - len(out))
        if not chunk:
            raise ConnectionError(f"closed after {len(out)} of {n} bytes")
        out += chunk
    return out


def test_fixture_decodes_as_the_documented_wire(session):
    """Each recorded request and answer parses per connector/tcpkv.py:9-17, with
    the blobs the seed regenerates and zlib CRC-32 (0 where unchecked)."""
    for e in session:
        c, s = e["client"], e["server"]
        if e["name"] == "stats":
            assert c == b"S"
            n = struct.unpack("<q", s[:8])[0]
            assert n == len(s) - 8 and json.loads(s[8:]) == e["json"]
            continue
        kb = e["key"].encode()
        assert c[1:5] == struct.pack("<i", len(kb)) and c[5:5 + len(kb)] == kb
        rest = c[5 + len(kb):]
        if e["name"].startswith("push"):
            assert c[:1] == b"P"
            n, crc = struct.unpack("<qI", rest[:12])
            data = rest[12:]
            assert n == len(data)
            if e["name"] == "push_bad_crc":
                assert data == bytes.fromhex(e["data"]) and crc == zlib.crc32(data) ^ 1
                assert s == b"ER"
                continue
            assert data == e["data"]
            assert crc == (0 if e["name"] == "push_unchecked" else zlib.crc32(data))
            assert s == b"OK"
        else:
            assert c[:1] == b"W" and rest == struct.pack("<i", e["wait_ms"])
            n, crc = struct.unpack("<qI", s[:12])
            if e["name"] == "take_absent":
                assert (n, crc, s[12:]) == (-1, 0, b"")
            else:
                assert s[12:] == e["data"] and n == len(e["data"])
                assert crc == (0 if e["name"] == "take_unchecked" else zlib.crc32(e["data"]))


def _replay_to_relay(port, session):
    with socket.create_connection(("127.0.0.1", port), timeout=10) as s:
        for e in session:
            s.sendall(e["client"])
            assert _recv(s, len(e["server"])) == e["server"], e["name"]


def test_native_relay_answers_as_the_reference_relay(session):
    srv = tcp.TcpKVServer(0, "127.0.0.1").start()
    try:
        _replay_to_relay(srv.wait_ready(), session)
        assert srv.stats == session[-1]["json"]
    finally:
        srv.stop()


def test_oracle_relay_answers_as_the_reference_relay(session):
    r = otcp.Relay()
    r.start()
    try:
        _replay_to_relay(r.port, session)
    finally:
        r.stop()


class _Script(threading.Thread):
    """A peer that expects the recorded requests in order (on whatever
    connections the client opens) and answers each with the recorded reply."""

    def __init__(self, exchanges):
        super().__init__(daemon=True)
        self.ex = list(exchanges)
        self.sock = socket.socket()
        self.sock.bind(("127.0.0.1", 0))
        self.sock.listen(4)
        self.sock.settimeout(10)
        self.port = self.sock.getsockname()[1]
        self.mismatch = []
        self.done = 0

    def run(self):
        try:
            while self.done < len(self.ex):
                c, _ = self.sock.accept()
                with c:
                    c.settimeout(10)
                    while self.done < len(self.ex):
                        e = self.ex[self.done]
                        try:
                            got = _recv(c, len(e["client"]))
                        except ConnectionError:
                            break                    # the client moved to another connection
                        if got != e["client"]:
                            self.mismatch.append((e["name"], got[:64].hex(), e["client"][:64].hex()))
                            return
                        c.sendall(e["server"])
                        self.done += 1
        except OSError as err:
            self.mismatch.append(("socket", repr(err), ""))
        finally:
            self.sock.close()


def test_native_client_speaks_as_the_reference_client(session, monkeypatch):
    client_side = [e for e in session if e["name"] != "push_bad_crc"]   # a raw-socket exchange
    peer = _Script(client_side)
    peer.start()
    c = tcp.TcpKVClient("127.0.0.1", peer.port)
    try:
        for e in client_side:
            name = e["name"]
            if name == "push":
                c.push(e["key"], e["data"])
            elif name == "push_unchecked":
                monkeypatch.setenv("AIRM_KV_TCP_CRC", "0")
                c.push(e["key"], e["data"])
                monkeypatch.delenv("AIRM_KV_TCP_CRC")
            elif name == "stats":
                assert c.stats() == e["json"]
            elif name in ("take", "take_unchecked"):
                if name == "take_unchecked":
                    monkeypatch.setenv("AIRM_KV_TCP_CRC", "0")
                assert bytes(c.take(e["key"], timeout=e["wait_ms"] / 1e3)) == e["data"]
                monkeypatch.delenv("AIRM_KV_TCP_CRC", raising=False)
            elif name == "take_absent":
                with pytest.raises(TimeoutError):
                    c.take(e["key"], timeout=e["wait_ms"] / 1e3)
            else:
                raise AssertionError(name)
    finally:
        c.close()
    peer.join(10)
    assert peer.mismatch == [] and peer.done == len(client_side)
