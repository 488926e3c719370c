"""The cross-node ``tcp`` KV transport over the native relay (librngdpd_net.so).

Same surfaces as the reference's connector/tcpkv.py and its TcpTransport
(connector/transport.py:104-151), same wire protocol, so either side can be
the reference's Python relay or client:

  TcpKVServer(port, host="0.0.0.0", ttl_s=None)   start() / wait_ready() -> port /
                                                  stop() / stats (dict) / ttl_s
  TcpKVClient(host, port)                         push / push_parts / take /
                                                  take_into / stats / close
  TcpTransport(remote=None, serve_port=None)      Transport: push / pull (+ push_parts /
                                                  pull_into for the device path);
                                                  remote or $AIRM_KV_TCP_ADDR
  parse_addr("host:port")

The relay, pooled client and CRC-32 are C++ (csrc/net/tcpkv.cpp): the GIL is
released for every network call, blobs are sent from and received into the
caller's buffers (pinned staging memory on the device path) without copies,
and the CRC runs at memory speed. AIRM_KV_TCP_CRC=0 skips computing it;
AIRM_KV_TCP_LOG=1 logs one line per blob (key, bytes, sha256 prefix, ms).

  python -m rngd_pd_amd.connector.tcp --port 5577      # a relay (no GPU needed)
"""
import argparse
import ctypes
import hashlib
import json
import os
import sys
import threading
import time

from .transport import Transport

_HERE = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB_PATH = os.path.join(_HERE, "librngdpd_net.so")
_LIB = None
_LOCK = threading.Lock()
ENOSPC, ETIMEDOUT, EIO = -28, -110, -5


class BlobTooLarge(ValueError):
    """The blob does not fit the caller's buffer; ``size`` is what it needs.
    The client keeps the blob: a take of the same key with a large enough
    buffer (or take()) returns it."""

    def __init__(self, key, size, cap):
        super().__init__(f"{key}: {size} bytes do not fit a {cap}-byte buffer")
        self.size = size


def _net():
    global _LIB
    with _LOCK:
        if _LIB is None:
            if not os.path.exists(LIB_PATH):
                raise RuntimeError(f"librngdpd_net.so is not built ({LIB_PATH}); run "
                                   f"__graft_entry__.build()")
            L = ctypes.CDLL(LIB_PATH)
            P, I, D, Z, I64 = ctypes.c_void_p, ctypes.c_int, ctypes.c_double, ctypes.c_size_t, \
                ctypes.c_int64
            sig = {
                "pdk_net_last_error": (ctypes.c_char_p, []),
                "pdk_crc32": (ctypes.c_uint32, [ctypes.c_uint32, P, Z]),
                "pdk_tcp_server_start": (I, [ctypes.c_char_p, I, D, ctypes.POINTER(P)]),
                "pdk_tcp_server_port": (I, [P]),
                "pdk_tcp_server_set_ttl": (I, [P, D]),
                "pdk_tcp_server_stats": (I64, [P, ctypes.c_char_p, Z]),
                "pdk_tcp_server_stop": (I, [P]),
                "pdk_tcp_client_open": (I, [ctypes.c_char_p, I, D, ctypes.POINTER(P)]),
                "pdk_tcp_client_idle": (I, [P]),
                "pdk_tcp_client_close": (I, [P]),
                "pdk_tcp_push": (I, [P, ctypes.c_char_p, ctypes.POINTER(P), ctypes.POINTER(Z), I,
                                     I]),
                "pdk_tcp_take": (I, [P, ctypes.c_char_p, I, P, Z, ctypes.POINTER(I64), I]),
                "pdk_tcp_stats": (I64, [P, ctypes.c_char_p, Z]),
            }
            for name, (res, args) in sig.items():
                f = getattr(L, name)
                f.restype, f.argtypes = res, args
            _LIB = L
        return _LIB


def _err():
    return _net().pdk_net_last_error().decode(errors="replace")


def crc32(data, crc=0):
    """zlib.crc32 semantics, native."""
    mv = memoryview(data).cast("B")
    buf = (ctypes.c_char * len(mv)).from_buffer_copy(mv) if mv.readonly else \
        (ctypes.c_char * len(mv)).from_buffer(mv)
    return _net().pdk_crc32(crc, ctypes.addressof(buf) if len(mv) else None, len(mv))


def _crc_on():
    return os.environ.get("AIRM_KV_TCP_CRC", "1") not in ("0", "false", "no")


def _address(buf):
    """(address, length, keepalive) of a bytes-like object without copying
    writable buffers; read-only ones (bytes) are referenced in place too."""
    mv = memoryview(buf).cast("B")
    n = len(mv)
    if n == 0:
        return None, 0, mv
    if mv.readonly:
        # bytes: its buffer is contiguous and immutable; ctypes can point at it.
        c = ctypes.c_char_p(bytes(mv) if not isinstance(buf, bytes) else buf)
        return ctypes.cast(c, ctypes.c_void_p).value, n, c
    arr = (ctypes.c_char * n).from_buffer(mv)
    return ctypes.addressof(arr), n, arr


class TcpKVServer:
    """The relay: an in-memory key -> bytes store behind a TCP port
    (connector/tcpkv.py:48-151). ``port`` 0 lets the OS pick; wait_ready()
    returns the port in use. Blobs nobody takes within ``ttl_s``
    ($AIRM_KV_TCP_TTL_S, 900) are dropped."""

    def __init__(self, port, host="0.0.0.0", ttl_s=None):
        self.port, self.host = port, host
        self._ttl = float(ttl_s if ttl_s is not None else os.environ.get("AIRM_KV_TCP_TTL_S", "900"))
        self._h = None

    def start(self):
        h = ctypes.c_void_p()
        rc = _net().pdk_tcp_server_start(self.host.encode(), int(self.port), self._ttl,
                                         ctypes.byref(h))
        if rc:
            raise OSError(f"tcpkv server: {_err()}")
        self._h = h
        self.port = _net().pdk_tcp_server_port(h)
        return self

    def wait_ready(self, timeout=5.0):
        if self._h is None:
            raise RuntimeError("TcpKVServer did not start")
        return self.port

    def is_alive(self):
        return self._h is not None

    @property
    def ttl_s(self):
        return self._ttl

    @ttl_s.setter
    def ttl_s(self, v):
        self._ttl = float(v)
        if self._h is not None:
            _net().pdk_tcp_server_set_ttl(self._h, self._ttl)

    @property
    def stats(self):
        buf = ctypes.create_string_buffer(1024)
        n = _net().pdk_tcp_server_stats(self._h, buf, len(buf))
        if n < 0:
            raise OSError(_err())
        return json.loads(buf.value.decode())

    def stop(self):
        if self._h is not None:
            _net().pdk_tcp_server_stop(self._h)
            self._h = None


class TcpKVClient:
    """Pooled persistent connections to one relay (connector/tcpkv.py:154-227).
    Safe to share between threads: each call borrows its own connection."""

    def __init__(self, host, port, connect_timeout=10.0):
        self.addr = (host, int(port))
        h = ctypes.c_void_p()
        rc = _net().pdk_tcp_client_open(host.encode(), int(port), float(connect_timeout),
                                        ctypes.byref(h))
        if rc:
            raise OSError(_err())
        self._h = h

    def idle_connections(self):
        return _net().pdk_tcp_client_idle(self._h)

    def push_parts(self, key, parts):
        keep = [_address(p) for p in parts]
        n = len(keep)
        ptrs = (ctypes.c_void_p * max(n, 1))(*[k[0] for k in keep])
        lens = (ctypes.c_size_t * max(n, 1))(*[k[1] for k in keep])
        rc = _net().pdk_tcp_push(self._h, key.encode(), ptrs, lens, n, int(_crc_on()))
        if rc == EIO:
            raise IOError(f"tcpkv push {key}: server rejected the blob (crc mismatch)")
        if rc:
            raise ConnectionError(_err())

    def push(self, key, data):
        self.push_parts(key, [data])

    def take_into(self, key, out, timeout=5.0):
        """Receive the blob into the writable buffer ``out``; returns its size.
        BlobTooLarge (a ValueError) when it does not fit."""
        addr, cap, keep = _address(out) if len(memoryview(out)) else (None, 0, None)
        n = ctypes.c_int64()
        rc = _net().pdk_tcp_take(self._h, key.encode(), max(0, int(timeout * 1e3)), addr, cap,
                                 ctypes.byref(n), int(_crc_on()))
        del keep
        if rc == ETIMEDOUT:
            raise TimeoutError(f"pull timeout: {key}")
        if rc == ENOSPC:
            raise BlobTooLarge(key, n.value, cap)
        if rc == EIO:
            raise IOError(f"tcpkv take {key}: crc mismatch on delivery")
        if rc:
            raise ConnectionError(_err())
        return n.value

    def take(self, key, timeout=5.0):
        """The blob pushed under ``key`` (bytearray), waiting up to ``timeout``;
        TimeoutError if it never came. Removes it from the relay."""
        buf = bytearray(1 << 20)
        try:
            n = self.take_into(key, buf, timeout)
        except BlobTooLarge as e:
            buf = bytearray(e.size)
            n = self.take_into(key, buf, timeout)
        del buf[n:]
        return buf

    def stats(self):
        buf = ctypes.create_string_buffer(4096)
        n = _net().pdk_tcp_stats(self._h, buf, len(buf))
        if n < 0:
            raise ConnectionError(_err())
        return json.loads(buf.value.decode())

    def close(self):
        if self._h is not None:
            _net().pdk_tcp_client_close(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def parse_addr(text, default_port=5577):
    """'host:port' or 'host' -> (host, port) (connector/tcpkv.py:230-233)."""
    host, _, port = text.strip().rpartition(":") if ":" in text else (text.strip(), "", "")
    return host, int(port or default_port)


class TcpTransport(Transport):
    """Cross-node KV through one relay (connector/transport.py:104-151).

    remote=(host, port), else $AIRM_KV_TCP_ADDR ("host:port"); serve_port=
    starts a relay in this process (and talks to it when no remote is named). select_transport("tcp") hands one shared instance to a
    process, so its connection pool outlives requests."""

    shared = True
    name = "tcp"

    def __init__(self, remote=None, serve_port=None):
        self.server = None
        if serve_port is not None:
            self.server = TcpKVServer(serve_port).start()
            serve_port = self.server.wait_ready()
        if remote is None and os.environ.get("AIRM_KV_TCP_ADDR"):
            remote = parse_addr(os.environ["AIRM_KV_TCP_ADDR"])
        if remote is None and serve_port is not None:
            remote = ("127.0.0.1", serve_port)
        self.remote = tuple(remote) if remote else None
        self._client = TcpKVClient(*self.remote) if self.remote else None

    def _need(self):
        if self._client is None:
            raise ValueError("tcp transport needs remote=(host, port) or AIRM_KV_TCP_ADDR=host:port")
        return self._client

    def push(self, key, buf):
        t0 = time.perf_counter()
        self._need().push(key, buf)
        self._log("push", key, buf, t0)

    def push_parts(self, key, parts):
        t0 = time.perf_counter()
        self._need().push_parts(key, parts)
        if os.environ.get("AIRM_KV_TCP_LOG", "0") not in ("0", ""):
            self._log("push", key, b"".join(bytes(p) for p in parts), t0)

    def pull(self, key, timeout=5.0):
        t0 = time.perf_counter()
        buf = self._need().take(key, timeout=timeout)     # the relay waits; no polling
        self._log("pull", key, buf, t0)
        return buf

    def pull_into(self, key, out, timeout=5.0):
        """Receive straight into ``out``; ValueError when it does not fit (the
        blob is then returned by the next pull of the key)."""
        t0 = time.perf_counter()
        n = self._need().take_into(key, out, timeout=timeout)
        if os.environ.get("AIRM_KV_TCP_LOG", "0") not in ("0", ""):
            self._log("pull", key, bytes(memoryview(out)[:n]), t0)
        return n

    @staticmethod
    def _log(op, key, buf, t0):
        if os.environ.get("AIRM_KV_TCP_LOG", "0") not in ("0", ""):
            sys.stdout.write(f"[kv-tcp] {op} {key} {len(buf)} "
                             f"{hashlib.sha256(bytes(buf)).hexdigest()[:16]} "
                             f"{(time.perf_counter() - t0) * 1e3:.2f}ms\n")
            sys.stdout.flush()

    def handshake_metadata(self):
        return {"tcp": "%s:%d" % self.remote} if self.remote else {}

    def close(self):
        if self._client:
            self._client.close()
        if self.server:
            self.server.stop()


def main(argv=None):
    ap = argparse.ArgumentParser(description="KV relay: holds pushed KV blobs until a pull takes them")
    ap.add_argument("--host", default="0.0.0.0")
    ap.add_argument("--port", type=int, default=int(os.environ.get("AIRM_KV_TCP_PORT", "5577")))
    ap.add_argument("--stats-every", type=float, default=60.0,
                    help="print counters every N s (0: never)")
    a = ap.parse_args(argv)
    srv = TcpKVServer(a.port, a.host).start()
    print(f"[tcpkv] relay on {a.host}:{srv.wait_ready()}", flush=True)
    last = None
    try:
        while srv.is_alive():
            time.sleep(a.stats_every or 3600)
            if a.stats_every:
                snap = srv.stats
                if snap != last:
                    print(f"[tcpkv] {json.dumps(snap)}", flush=True)
                    last = snap
    except KeyboardInterrupt:
        srv.stop()


if __name__ == "__main__":
    main()
