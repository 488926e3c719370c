"""rm-core ``airm.kv_transports`` adapters: the ``shm`` and ``tcp`` KV paths
(the reference's airm.py:57-271).

ShmTransport and TcpTransport are both rm-core KVTransports (plan / submit /
wait / take / close / conformance_case) and the connector's push/pull
Transports, so ``select_transport(name)`` hands the workers the same object the
registry names. Entry points: ``airm.kv_transports: shm =
rngd_pd_amd.airm:ShmTransport`` and ``tcp = rngd_pd_amd.airm:TcpTransport``.
Both are host-staging paths between two host-memory tiers (shm on one
machine, tcp between any two through a relay).
"""
import collections
import os
import threading
import time
import uuid

import numpy as np

from .connector import tcp as _tcp
from .connector import transport as _kv
from .paths import SHM_ROOT
from .rm_compat import (ContractError, KVLayout, Measurement, MemoryTier,  # noqa: F401
                        TransferHandle, TransferPlan, TransferResult, TransportError)

COMPONENT = "rngd-pd"
WIRE_DTYPES = ("bf16", "fp16")          # what the wire carries, 2 bytes an element


class _KeyedKV:
    """rm-core KVTransport methods over a key -> bytes transport (airm.py:57-134).

    A subclass sets ``name`` and ``SCOPE``, implements supports() and _detail(),
    and provides _fetch(key, timeout) (the bytes, TimeoutError if absent) and
    _consume(key) (the bytes once more, then removed).
    """

    def _init_kv(self):
        self._pending = {}                  # handle token -> (plan, key, started)
        self._delivered = {}                # (request id, tokens) -> key waited but not taken
        self._lock = threading.Lock()
        self.measurements = collections.deque(maxlen=1024)

    def _sent(self, key):
        """Hook: submit() published ``key``."""

    def plan(self, request_id, src, dst, src_layout, dst_layout, tokens):
        if not self.supports(src, dst):
            raise TransportError(f"{self.name}: {self.SCOPE}, "
                                 f"not {src.kind}:{src.name} -> {dst.kind}:{dst.name}")
        src_layout.validate()
        dst_layout.validate()
        if src_layout != dst_layout:
            raise TransportError(f"{self.name}: src and dst layouts differ; convert in the model adapter")
        if src_layout.dtype not in WIRE_DTYPES:
            raise TransportError(f"{self.name}: wire carries {WIRE_DTYPES}, not {src_layout.dtype}")
        start, end = tokens
        if not 0 <= start < end:
            raise TransportError(f"{self.name}: bad token range {tokens}")
        return TransferPlan(request_id, src.validate(), dst.validate(), src_layout, dst_layout,
                            (start, end), (end - start) * src_layout.bytes_per_token(),
                            detail=dict(self._detail(), wire=src_layout.dtype))

    def submit(self, plan, kv=None):
        """kv: the range's KV as (end-start)*bytes_per_token/2 elements; zeros if omitted."""
        n = plan.nbytes // 2
        if kv is None:
            kv = np.zeros(n, np.float32)
        elif np.asarray(kv).size != n:
            raise ContractError(f"{self.name}: kv has {np.asarray(kv).size} elements, plan needs {n}")
        token = uuid.uuid4().hex
        key = f"{plan.request_id}/{plan.dst.name}/{plan.tokens[0]}-{plan.tokens[1]}.{token[:8]}"
        started = time.perf_counter()
        self.push(key, _kv.ser(np.asarray(kv, np.float32), wire=plan.detail.get("wire", "bf16")))
        with self._lock:
            self._pending[token] = (plan, key, started)
        self._sent(key)
        return TransferHandle(plan.request_id, self.name, token)

    def wait(self, handle, timeout_s):
        """Never raises for a missing or short segment: ok=False instead."""
        with self._lock:
            entry = self._pending.pop(handle.token, None)
        if entry is None:
            raise TransportError(f"{self.name}: unknown or already-waited handle {handle.token}")
        plan, key, started = entry
        try:
            got = _kv.deser(self._fetch(key, timeout_s)).size * 2
        except TimeoutError as e:
            return TransferResult(plan.request_id, False, 0, time.perf_counter() - started, str(e))
        seconds = time.perf_counter() - started
        if got != plan.nbytes:
            return TransferResult(plan.request_id, False, got, seconds,
                                  f"segment holds {got} bytes, plan moved {plan.nbytes}")
        self.measurements.append(Measurement(
            "kv_transfer_ms", seconds * 1e3,
            {"component": COMPONENT, "kv_transport": self.name}).validate())
        with self._lock:
            self._delivered[(plan.request_id, plan.tokens)] = key
        return TransferResult(plan.request_id, True, plan.nbytes, seconds)

    def take(self, plan):
        """The delivered KV for ``plan`` as float32, removing it."""
        with self._lock:
            key = self._delivered.pop((plan.request_id, plan.tokens), None)
        if key is None:
            raise TransportError(f"{self.name}: nothing delivered for {plan.request_id} {plan.tokens}")
        return _kv.deser(self._consume(key))


class ShmTransport(_KeyedKV, _kv.ShmTransport):
    """KV between two host-memory tiers on one machine, through /dev/shm.

    root defaults to $PD_SHM_ROOT, else /dev/shm/rngd_kv_cluster; both sides must
    see the same directory. Constructing creates nothing: the directory is made
    on the first write. wait() never falls back to another path.
    """

    name = "shm"
    SCOPE = "only host-dram -> host-dram on one machine"

    def __init__(self, root=None):
        self.root = str(root or os.environ.get("PD_SHM_ROOT") or SHM_ROOT)
        self._written = set()
        self._init_kv()

    def push(self, key, buf):
        os.makedirs(self.root, exist_ok=True)
        super().push(key, buf)

    def push_parts(self, key, parts):
        os.makedirs(self.root, exist_ok=True)
        super().push_parts(key, parts)

    def supports(self, src, dst):
        return src.kind == "host-dram" and dst.kind == "host-dram" and src.name != dst.name

    def _detail(self):
        return {"root": self.root}

    def _sent(self, key):
        with self._lock:
            self._written.add(key)

    def _fetch(self, key, timeout):
        return self.pull(key, timeout=timeout)

    def _consume(self, key):
        buf = self.pull(key, timeout=0)
        self._unlink(key)
        return buf

    def close(self):
        """Remove the keys this instance published (and its conformance directory)."""
        with self._lock:
            keys, self._written = self._written, set()
            self._pending.clear()
            self._delivered.clear()
        for key in keys:
            self._unlink(key)
        if os.path.basename(self.root).startswith("rngd_kv_conformance."):
            try:
                os.rmdir(self.root)
            except OSError:
                pass

    def _unlink(self, key):
        try:
            os.unlink(self._path(key))
        except FileNotFoundError:
            pass
        with self._lock:
            self._written.discard(key)

    def conformance_case(self):
        """Two host tiers sharing /dev/shm, in a private directory next to the
        serving root so a check never touches live handoff files."""
        from .rm_compat import NoHardware
        self.root = os.path.join(os.path.dirname(self.root.rstrip("/")) or "/dev/shm",
                                 f"rngd_kv_conformance.{os.getuid()}.{os.getpid()}")
        try:
            os.makedirs(self.root, exist_ok=True)
            probe = os.path.join(self.root, f".probe.{os.getpid()}")
            open(probe, "wb").close()
            os.unlink(probe)
        except OSError as e:
            raise NoHardware(f"shm root {self.root} is not writable: {e}") from e
        return (MemoryTier("shm-prefill", "host-dram", 1 << 30),
                MemoryTier("shm-decode", "host-dram", 1 << 30),
                KVLayout(num_layers=2, num_kv_heads=2, head_dim=8, dtype="bf16"))


class TcpTransport(_KeyedKV, _tcp.TcpTransport):
    """KV between two host-memory tiers on any two machines, through one relay
    (the native librngdpd_net.so; airm.py:224-271 of the reference).

    Keyword arguments: remote -- (host, port) of the relay both sides use
    (default $AIRM_KV_TCP_ADDR), serve_port -- also run a relay in this process.
    Every blob carries a CRC-32 checked by the relay and by the receiver, so
    wait() is ok only for the bytes submit() sent. The relay hands a blob out
    once, so wait() keeps it for take()."""

    name = "tcp"
    SCOPE = "only host-dram -> host-dram"

    def __init__(self, remote=None, serve_port=None):
        _tcp.TcpTransport.__init__(self, remote=remote, serve_port=serve_port)
        self._held = {}
        self._init_kv()

    def supports(self, src, dst):
        return src.kind == "host-dram" and dst.kind == "host-dram" and src.name != dst.name

    def _detail(self):
        return {"server": "%s:%d" % self.remote if self.remote else None}

    def _fetch(self, key, timeout):
        buf = self.pull(key, timeout=timeout)
        with self._lock:
            self._held[key] = buf
        return buf

    def _consume(self, key):
        with self._lock:
            return self._held.pop(key)

    def close(self):
        with self._lock:
            self._pending.clear()
            self._delivered.clear()
            self._held.clear()
        _tcp.TcpTransport.close(self)

    def conformance_case(self):
        """Two host tiers and a relay on a free loopback port in this process."""
        if self.remote is None:
            _tcp.TcpTransport.__init__(self, serve_port=0)
        return (MemoryTier("tcp-prefill", "host-dram", 1 << 30),
                MemoryTier("tcp-decode", "host-dram", 1 << 30),
                KVLayout(num_layers=2, num_kv_heads=2, head_dim=8, dtype="bf16"))
