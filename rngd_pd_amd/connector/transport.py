"""Key -> bytes KV transports of the connector (the reference's connector/transport.py).

  Transport         push(key, buf) / pull(key, timeout) -> bytes / close()   (:46-60)
  InProcTransport   dict in one process (tests)                               (:63-77)
  ShmTransport      /dev/shm files: write tmp.<pid>, fsync, rename (atomic
                    publish); pull polls every millisecond                   (:80-101)
                    + push_parts / pull_into: the same files written from and
                    read into pinned staging buffers without intermediate copies
  FencedTransport   a tier-to-tier rm-core transport behind push/pull        (:238-289)
  select_transport  by name: $AIRM_KV_TRANSPORT, default "shm"; no fallback  (:292-350)

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

    def discard(self, key):
        with self._lock:
            self._store.pop(key, None)

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

    def discard(self, key):
        """Remove ``key``'s file if it is there (a consumer is done with it)."""
        try:
            os.unlink(self._path(key))
        except FileNotFoundError:
            pass

    def discard_request(self, req_id):
        """Remove every file of request ``req_id`` ("<req_id>__..."): the consumer's
        purge once a request's KV is loaded (serving/cluster.py:461-466).
        Returns the number of files removed."""
        prefix = req_id.replace("/", "__") + "__"
        n = 0
        try:
            names = os.listdir(self.root)
        except FileNotFoundError:
            return 0
        for f in names:
            if f.startswith(prefix):
                try:
                    os.unlink(os.path.join(self.root, f))
                    n += 1
                except FileNotFoundError:
                    pass
        return n

    def close(self):
        pass                     # files persist for the peer; the consumer removes them


class NixlTransport(Transport):
    """Cross-device NIXL path: not part of this package; fails loudly, never falls back."""

    def __init__(self, *a, **kw):
        raise NotImplementedError("NIXL transport is not available in this package; "
                                  "use the shm transport (same host)")

    def push(self, key, buf):
        raise NotImplementedError

    def pull(self, key, timeout=5.0):
        raise NotImplementedError


class FencedTransport(Transport):
    """The connector's key -> bytes contract over an rm-core tier-to-tier
    transport (one that moves KV between memory tiers itself and knows nothing
    of keys). push() plans and submits one transfer per key; pull() blocks
    until that key has been pushed, then on its transfer's completion fence,
    and only then returns the bytes. A failed fence raises TransportError, a
    second push of a key that was not pulled yet raises ValueError. Handles are
    process-local, so both ends live in one process (connector/transport.py:238-289).

    Pushes and pulls meet at a condition variable: a pull sleeps until the
    key's push has submitted (or the timeout passes) instead of polling."""

    _SUBMITTING = object()               # a push holds the key while it submits

    def __init__(self, impl, src=None, dst=None):
        from ..rm_compat import KVLayout, MemoryTier
        self.impl = impl
        self.name = impl.name
        self.src = src or MemoryTier("prefill", "host-dram", 1 << 40)
        self.dst = dst or MemoryTier("decode", "host-dram", 1 << 40)
        # One "token" per 2 bytes (1 layer x 1 head x 1 dim of int8 K and V),
        # so a plan of ceil(n / 2) tokens covers an n-byte blob.
        self._layout = KVLayout(num_layers=1, num_kv_heads=1, head_dim=1, dtype="int8")
        self._cv = threading.Condition()
        self._fences = {}                # key -> (handle, buf), or _SUBMITTING

    def push(self, key, buf):
        tokens = (0, max(1, (len(buf) + 1) // 2))
        plan = self.impl.plan(key, self.src, self.dst, self._layout, self._layout, tokens)
        with self._cv:
            if key in self._fences:
                raise ValueError(f"{self.name}: key {key!r} is still waiting for its pull")
            self._fences[key] = self._SUBMITTING
        try:
            handle = self.impl.submit(plan)
        except BaseException:
            with self._cv:
                del self._fences[key]
            raise
        with self._cv:
            self._fences[key] = (handle, buf)
            self._cv.notify_all()

    def pull(self, key, timeout=5.0):
        from ..rm_compat import TransportError
        deadline = time.monotonic() + timeout
        with self._cv:
            if not self._cv.wait_for(lambda: isinstance(self._fences.get(key), tuple), timeout):
                raise TimeoutError(f"pull timeout: {key}")
            handle, buf = self._fences[key]
        try:
            res = self.impl.wait(handle, timeout_s=max(0.0, deadline - time.monotonic()))
        finally:
            with self._cv:
                self._fences.pop(key, None)      # a handle is waited at most once
        if not res.ok:
            raise TransportError(f"{self.name}: the transfer of {key!r} did not complete: "
                                 f"{res.error}")
        return buf

    def close(self):
        _SELECTOR.forget(self)
        self.impl.close()


class _Selector:
    """Transport names -> implementations, resolved once per process.

    Resolution: rm-core's ``airm.kv_transports`` registry when rm-core is
    installed, then this package's own table; without rm-core, only the own
    table. Anything else is a KeyError -- there is no fallback path. A
    tier-to-tier implementation is wrapped in one FencedTransport per process
    (both ends must share its handles); an implementation that declares
    ``shared`` (it holds connections) is one instance per process; every other
    is made anew per call (connector/transport.py:292-350)."""

    OWN = {"shm": "rngd_pd_amd.airm:ShmTransport",
           "tcp": "rngd_pd_amd.airm:TcpTransport",              # native relay client
           "ipc": "rngd_pd_amd.connector.ipc:IpcTransport"}     # same-GPU frames in HBM
    ABSENT = ("nixl", "nixl-ucx")       # vendor P2P paths this package does not provide

    def __init__(self):
        self._lock = threading.RLock()
        self._factories = {}             # name -> class
        self._held = {}                  # name -> the instance kept for the process

    def reset(self):
        """Forget every resolution and held instance (tests)."""
        with self._lock:
            self._factories.clear()
            self._held.clear()

    def held(self):
        with self._lock:
            return dict(self._held)

    def forget(self, instance):
        with self._lock:
            for name in [n for n, t in self._held.items() if t is instance]:
                del self._held[name]

    def _construct(self, name, kw):
        cls = self._factories.get(name)
        if cls is not None:
            return cls(**kw)
        from .. import rm_compat
        impl = None
        if rm_compat.registry is not None:
            try:
                impl = rm_compat.registry.load("airm.kv_transports", name, **kw)
            except KeyError:
                impl = None
        if impl is None:
            target = self.OWN.get(name)
            if target is None:
                if name in self.ABSENT:
                    raise KeyError(f"kv transport {name!r} is a vendor P2P path this package "
                                   f"does not provide")
                hint = "" if rm_compat.registry is not None else " (rm-core is not installed)"
                raise KeyError(f"no kv transport named {name!r}{hint}")
            import importlib
            module, attr = target.split(":")
            impl = getattr(importlib.import_module(module), attr)(**kw)
        self._factories[name] = type(impl)
        return impl

    def select(self, name, kw):
        with self._lock:
            if not kw and name in self._held:
                return self._held[name]
            impl = self._construct(name, kw)
            if isinstance(impl, Transport):
                if not kw and getattr(impl, "shared", False):
                    self._held[name] = impl
                return impl
            fenced = FencedTransport(impl)
            if not kw:
                self._held[name] = fenced
            return fenced


_SELECTOR = _Selector()


def reset_selection():
    """Drop the process's resolved transports (for tests that change the environment)."""
    _SELECTOR.reset()


def select_transport(name=None, **kw) -> Transport:
    """The connector's KV path by name: ``name``, else $AIRM_KV_TRANSPORT, else "shm".

    Keyword arguments go to the implementation's constructor (and then bypass
    the per-process instances). An unknown name raises KeyError."""
    return _SELECTOR.select(name or os.environ.get("AIRM_KV_TRANSPORT") or "shm", kw)


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
