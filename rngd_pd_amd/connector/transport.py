"""Key -> bytes KV transports of the connector (the reference's connector/transport.py).

  Transport         push(key, buf) / pull(key, timeout) -> bytes / close()   (:46-60)
  InProcTransport   dict in one process (tests)                               (:63-77)
  ShmTransport      /dev/shm files: write tmp.<pid>, fsync, rename (atomic
                    publish); pull polls every millisecond                   (:80-101)
                    + push_parts / pull_into: the same files written from and
                    read into pinned staging buffers without intermediate copies
  FencedTransport   a tier-to-tier rm-core transport behind push/pull        (:238-289)
  select_transport  by name: $AIRM_KV_TRANSPORT, default "shm"; no fallback  (:330-350)

  tcp               the cross-node relay transport, native (connector/tcp.py)
  ipc               same-GPU frames through hipIpc handles (connector/ipc.py)

The nixl-ucx / nixl transports of the reference (vendor P2P paths) are
outside this package; selecting them raises.
"""
import os
import threading
import time
from abc import ABC, abstractmethod

from . import wire as _wire
from .wire import deser  # noqa: F401  (the reference exports it from this module)

# Wire format of ser() when no wire is named: "fp16" by default as in the
# reference (:27); the serving workers set it to "bf16" (bit-exact for
# bf16-valued KV).
WIRE = "fp16"


def ser(arr, wire=None):
    """connector/transport.py:29-37, reading this module's WIRE default."""
    return _wire.ser(arr, wire or WIRE)


class Transport(ABC):
    """Key -> bytes KV transport. push may buffer; pull blocks until present."""

    @abstractmethod
    def push(self, key: str, buf: bytes) -> None: ...

    @abstractmethod
    def pull(self, key: str, timeout: float = 5.0) -> bytes: ...

    def close(self) -> None:
        pass

    def handshake_metadata(self) -> dict:
        """What a remote peer needs to reach this end (none for host transports)."""
        return {}

    def set_remote_handshake(self, meta: dict) -> None:
        pass


class InProcTransport(Transport):
    """In-process shared dict (unit tests, single process)."""

    def __init__(self):
        self._store = {}
        self._lock = threading.Lock()

    def push(self, key, buf):
        with self._lock:
            self._store[key] = bytes(buf) if not isinstance(buf, bytes) else buf

    def push_parts(self, key, parts):
        self.push(key, b"".join(bytes(p) for p in parts))

    def pull(self, key, timeout=5.0):
        t0 = time.time()
        while True:
            with self._lock:
                if key in self._store:
                    return self._store[key]
            if time.time() - t0 > timeout:
                raise TimeoutError(f"pull timeout: {key}")
            time.sleep(0.001)

    def close(self):
        self._store.clear()


def _write_all(fd, parts):
    """os.writev until every byte of ``parts`` is written."""
    views = [memoryview(p).cast("B") for p in parts if len(p)]
    while views:
        n = os.writev(fd, views)
        while n and views:
            if n >= len(views[0]):
                n -= len(views[0])
                views.pop(0)
            else:
                views[0] = views[0][n:]
                n = 0


class ShmTransport(Transport):
    """/dev/shm file store, cross-process on one host.

    A key maps to ``root/key.replace("/", "__")``. push writes ``<file>.tmp.<pid>``,
    flushes, fsyncs and renames it into place, so pull never sees a partial file.
    """

    def __init__(self, root="/dev/shm/rngd_kv"):
        self.root = str(root)
        os.makedirs(self.root, exist_ok=True)

    def _path(self, key):
        return os.path.join(self.root, key.replace("/", "__"))

    def push(self, key, buf):
        self.push_parts(key, [buf])

    def push_parts(self, key, parts):
        """Publish the concatenation of ``parts`` under ``key`` (no join copy)."""
        p = self._path(key)
        tmp = p + f".tmp.{os.getpid()}"
        fd = os.open(tmp, os.O_WRONLY | os.O_CREAT | os.O_TRUNC, 0o644)
        try:
            _write_all(fd, parts)
            os.fsync(fd)
        finally:
            os.close(fd)
        os.rename(tmp, p)

    def _wait(self, key, timeout):
        p = self._path(key)
        t0 = time.time()
        while not os.path.exists(p):
            if time.time() - t0 > timeout:
                raise TimeoutError(f"pull timeout: {key}")
            time.sleep(0.001)
        return p

    def pull(self, key, timeout=5.0):
        with open(self._wait(key, timeout), "rb") as f:
            return f.read()

    def pull_size(self, key, timeout=5.0):
        """Wait for ``key`` and return its size in bytes."""
        return os.path.getsize(self._wait(key, timeout))

    def pull_into(self, key, out, timeout=5.0):
        """Read ``key`` into the writable buffer ``out``; returns the byte count."""
        p = self._wait(key, timeout)
        mv = memoryview(out).cast("B")
        size = os.path.getsize(p)
        if size > len(mv):
            raise ValueError(f"{key}: {size} bytes do not fit a {len(mv)}-byte buffer")
        fd = os.open(p, os.O_RDONLY)
        try:
            got = 0
            while got < size:
                n = os.readv(fd, [mv[got:size]])
                if n == 0:
                    break
                got += n
        finally:
            os.close(fd)
        if got != size:
            raise IOError(f"{key}: short read ({got} of {size} bytes)")
        return size

    def close(self):
        pass                     # files persist for the peer; the consumer removes them


class NixlTransport(Transport):
    """Cross-device NIXL path: not part of this package; fails loudly, never falls back."""

    def __init__(self, *a, **kw):
        raise NotImplementedError("NIXL transport is not available in this build; "
                                  "use the shm transport (same host)")

    def push(self, key, buf):
        raise NotImplementedError

    def pull(self, key, timeout=5.0):
        raise NotImplementedError


class FencedTransport(Transport):
    """The connector's key -> bytes contract over an rm-core tier-to-tier transport.

    push() plans and submits one transfer per key; pull() waits on that transfer's
    fence and only then returns the bytes. A failed fence raises TransportError,
    a key pushed twice before its pull raises ValueError. Handles are process-local.
    """

    def __init__(self, impl, src=None, dst=None):
        from ..rm_compat import KVLayout, MemoryTier
        self.impl = impl
        self.name = impl.name
        self.src = src or MemoryTier("prefill", "host-dram", 1 << 40)
        self.dst = dst or MemoryTier("decode", "host-dram", 1 << 40)
        self._layout = KVLayout(num_layers=1, num_kv_heads=1, head_dim=1, dtype="int8")
        self._pending = {}
        self._lock = threading.Lock()

    def push(self, key, buf):
        n = len(buf)
        plan = self.impl.plan(key, self.src, self.dst, self._layout, self._layout,
                              (0, max(1, (n + 1) // 2)))
        with self._lock:
            if key in self._pending:
                raise ValueError(f"{self.name}: {key} pushed twice before it was pulled")
            self._pending[key] = None
        handle = self.impl.submit(plan)
        with self._lock:
            self._pending[key] = (handle, buf)

    def pull(self, key, timeout=5.0):
        from ..rm_compat import TransportError
        t0 = time.time()
        while True:
            with self._lock:
                entry = self._pending.get(key)
            if entry is not None:
                break
            if time.time() - t0 > timeout:
                raise TimeoutError(f"pull timeout: {key}")
            time.sleep(0.001)
        handle, buf = entry
        try:
            res = self.impl.wait(handle, timeout_s=max(0.0, timeout - (time.time() - t0)))
        finally:
            with self._lock:
                self._pending.pop(key, None)
        if not res.ok:
            raise TransportError(f"{self.name}: transfer {key} failed: {res.error}")
        return buf

    def close(self):
        with _LOCK:
            for k in [k for k, v in _FENCED.items() if v is self]:
                del _FENCED[k]
        self.impl.close()


# Our own adapters, used when the registry has no entry point of that name.
_OWN = {"shm": "rngd_pd_amd.airm:ShmTransport",
        "tcp": "rngd_pd_amd.airm:TcpTransport",            # native relay (librngdpd_net.so)
        "ipc": "rngd_pd_amd.connector.ipc:IpcTransport"}   # same-GPU frames in HBM
_NOT_HERE = ("nixl-ucx", "nixl")
_CLASSES = {}          # name -> implementation class, resolved once per process
_FENCED = {}           # name -> the process's one FencedTransport
_SHARED = {}           # name -> the process's one instance of a connection-holding transport
_LOCK = threading.Lock()


def _resolve(name, kw):
    cls = _CLASSES.get(name)
    if cls is not None:
        return cls(**kw)
    from .. import rm_compat
    try:
        impl = rm_compat.registry.load("airm.kv_transports", name, **kw)
    except KeyError:
        if name in _NOT_HERE:
            raise KeyError(f"AIRM_KV_TRANSPORT={name!r} is a cross-node transport this "
                           f"package does not provide")
        if name not in _OWN:
            raise
        import importlib
        mod, obj = _OWN[name].split(":")
        impl = getattr(importlib.import_module(mod), obj)(**kw)
    _CLASSES[name] = type(impl)
    return impl


def select_transport(name=None, **kw) -> Transport:
    """The connector's KV path by name: ``name``, else $AIRM_KV_TRANSPORT, else "shm".

    An implementation that speaks push/pull is returned as is (one shared instance
    per process if it declares ``shared``); a tier-to-tier transport is wrapped in
    FencedTransport. An unknown name raises KeyError: there is no fallback.
    """
    name = name or os.environ.get("AIRM_KV_TRANSPORT") or "shm"
    with _LOCK:
        if not kw and name in _FENCED:
            return _FENCED[name]
        if not kw and name in _SHARED:
            return _SHARED[name]
        impl = _resolve(name, kw)
        if isinstance(impl, Transport):
            if not kw and getattr(impl, "shared", False):
                _SHARED[name] = impl
            return impl
        t = FencedTransport(impl)
        if not kw:
            _FENCED[name] = t
        return t


def make_transport(backend="shm", **kw) -> Transport:
    """Factory by backend name: inproc, shm, ipc, tcp, nixl (raises)."""
    b = backend.lower()
    if b == "inproc":
        return InProcTransport()
    if b == "shm":
        return ShmTransport(**kw)
    if b == "ipc":
        from .ipc import IpcTransport
        return IpcTransport(**kw)
    if b == "nixl":
        return NixlTransport(**kw)
    if b == "tcp":
        from .tcp import TcpTransport
        return TcpTransport(**kw)
    if b == "nixl-ucx":
        raise NotImplementedError(f"{backend} is a cross-node transport this package does not provide")
    raise ValueError(f"unknown transport backend: {backend}")
