"""Records the reference's tcp KV wire as byte fixtures (tests/golden/tcp_wire.json).

Run from the repo root in the build container, where the reference is on disk:

    python tests/golden/make_tcp_golden.py [/path/to/reference]

It loads the reference's stdlib-only relay and client module,
src/rngd_pd/connector/tcpkv.py (wire at :9-17, relay :48-151, client
:154-227), by file path, starts its TcpKVServer on loopback and drives its
TcpKVClient through a recording proxy. Every exchange is one request and its
complete reply, so the bytes each direction carried between two calls are that
exchange's. Exchanges the client cannot produce (a push whose CRC is wrong)
go through the same proxy from a raw socket. The fixture holds, per exchange,
its name, what the client sent and what the relay answered (hex), in order,
plus the blobs' seeds and sizes; it is data, and no run of the tests needs the
reference: the tests replay it against the native relay and client and against
the oracle's protocol restatement.
"""
import importlib.util
import json
import os
import socket
import struct
import sys
import threading
import time
import zlib

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))


def load_reference(root):
    path = os.path.join(root, "src", "rngd_pd", "connector", "tcpkv.py")
    spec = importlib.util.spec_from_file_location("reference_tcpkv", path)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


class Tap:
    """Loopback proxy in front of one upstream port: every byte is recorded
    before it is forwarded, so when a synchronous call returns, both
    directions of its exchange are in the record."""

    def __init__(self, upstream):
        self.upstream = upstream
        self.lock = threading.Lock()
        self.sent, self.got = bytearray(), bytearray()
        self.sock = socket.socket()
        self.sock.bind(("127.0.0.1", 0))
        self.sock.listen(8)
        self.port = self.sock.getsockname()[1]
        threading.Thread(target=self._accept, daemon=True).start()

    def _accept(self):
        while True:
            try:
                down, _ = self.sock.accept()
            except OSError:
                return
            up = socket.create_connection(("127.0.0.1", self.upstream))
            for a, b, rec in ((down, up, self.sent), (up, down, self.got)):
                threading.Thread(target=self._pump, args=(a, b, rec), daemon=True).start()

    def _pump(self, src, dst, rec):
        while True:
            try:
                chunk = src.recv(1 << 16)
            except OSError:
                chunk = b""
            if not chunk:
                for s in (src, dst):
                    try:
                        s.shutdown(socket.SHUT_RDWR)
                    except OSError:
                        pass
                return
            with self.lock:
                rec += chunk
            dst.sendall(chunk)

    def cut(self, settle=0.05):
        time.sleep(settle)                      # a reply already delivered is already recorded
        with self.lock:
            out = (bytes(self.sent), bytes(self.got))
            self.sent.clear()
            self.got.clear()
        return out


def main():
    ref_root = sys.argv[1] if len(sys.argv) > 1 else "/root/reference"
    ref = load_reference(ref_root)
    srv = ref.TcpKVServer(0, "127.0.0.1")
    srv.start()
    port = srv.wait_ready()
    tap = Tap(port)
    cli = ref.TcpKVClient("127.0.0.1", tap.port)
    rng = np.random.default_rng(20261019)
    blob_k, blob_v = rng.bytes(4096), rng.bytes(1000)
    ex = []

    def record(name, **meta):
        sent, got = tap.cut()
        ex.append({"name": name, "client": sent.hex(), "server": got.hex(), **meta})

    cli.push("req-0/layer.0/k", blob_k)
    record("push", key="req-0/layer.0/k", blob="k")
    cli.push("req-0/layer.0/v", blob_v)
    record("push", key="req-0/layer.0/v", blob="v")
    stats = cli.stats()
    record("stats", json=stats)
    assert bytes(cli.take("req-0/layer.0/k", timeout=1.0)) == blob_k
    record("take", key="req-0/layer.0/k", wait_ms=1000, blob="k")
    try:
        cli.take("req-0/layer.9/k", timeout=0.05)
        raise AssertionError("take of an absent key returned")
    except TimeoutError:
        pass
    record("take_absent", key="req-0/layer.9/k", wait_ms=50)
    # A push whose CRC does not match its data: the relay answers ER and keeps nothing.
    bad = b"payload"
    kb = b"req-0/layer.1/k"
    with socket.create_connection(("127.0.0.1", tap.port)) as s:
        s.sendall(b"P" + struct.pack("<i", len(kb)) + kb +
                  struct.pack("<qI", len(bad), zlib.crc32(bad) ^ 1) + bad)
        assert s.recv(2) == b"ER"
    record("push_bad_crc", key=kb.decode(), data=bad.hex())
    os.environ["AIRM_KV_TCP_CRC"] = "0"         # crc 0 on the wire: unchecked
    cli.push("req-0/layer.2/k", blob_v[:333])
    record("push_unchecked", key="req-0/layer.2/k", blob="v", length=333)
    assert bytes(cli.take("req-0/layer.2/k", timeout=1.0)) == blob_v[:333]
    record("take_unchecked", key="req-0/layer.2/k", wait_ms=1000, blob="v", length=333)
    del os.environ["AIRM_KV_TCP_CRC"]
    cli.push("req-1/layer.0/k", b"")
    record("push", key="req-1/layer.0/k", blob="empty")
    assert bytes(cli.take("req-1/layer.0/k", timeout=1.0)) == b""
    record("take", key="req-1/layer.0/k", wait_ms=1000, blob="empty")
    record_stats = cli.stats()
    record("stats", json=record_stats)
    cli.close()
    srv.stop()
    fixture = {
        "source": "connector/tcpkv.py (TcpKVServer, TcpKVClient) over loopback",
        "blobs": {"seed": 20261019, "k": 4096, "v": 1000,
                  "generator": "np.random.default_rng(seed).bytes(k) then .bytes(v)"},
        "exchanges": ex,
    }
    with open(os.path.join(HERE, "tcp_wire.json"), "w") as f:
        json.dump(fixture, f, indent=1)
        f.write("\n")
    print(f"{len(ex)} exchanges, {sum(len(e['client']) + len(e['server']) for e in ex) // 2} bytes")


if __name__ == "__main__":
    main()
