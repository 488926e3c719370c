"""rm-core ``airm.kv_transports`` adapters for the ``shm`` and ``tcp`` KV paths.

The contract is rm-core v0.1.1's KVTransport as the reference's adapter meets
it (airm.py:57-271 and tests/test_airm.py:76-212):

  plan(request_id, src, dst, src_layout, dst_layout, (start, end))
      -> TransferPlan(nbytes = (end - start) * layout.bytes_per_token(),
                      detail = {route..., "wire": dtype}); TransportError for an
      unsupported tier pair, differing layouts, a dtype the 2-byte wire cannot
      carry (bf16 and fp16 only) or an empty range
  submit(plan, kv=None) -> TransferHandle; kv holds nbytes / 2 elements
      (ContractError otherwise, zeros when omitted); the segment is published
      under "{request}/{dst.name}/{start}-{end}.{uuid8}"
  wait(handle, timeout_s) -> TransferResult; ok=False for a missing, short or
      unreadable segment (never an exception), TransportError for a handle
      that is unknown or already waited; a good wait appends
      Measurement("kv_transfer_ms", ms, {component, kv_transport})
  take(plan) -> the delivered KV as float32, consumed
  close()  discards what this instance published and nobody consumed
  conformance_case() -> (src tier, dst tier, KVLayout(2, 2, 8, "bf16"))

Both adapters are also the connector's key -> bytes Transports, so
select_transport(name) hands the serving workers the object the registry names.

Design. Each adapter keeps a _Ledger of its transfers. A _Transfer records the
plan, the key it was published under and when; it is "in flight" from submit()
until wait(), and "landed" from a good wait() until take(). wait() fetches the
segment and decodes it once (the restricted unpickler of connector.wire);
the landed transfer holds the float32 array, so take() only hands it over and
discards the segment. A failed wait() discards the segment at once. What the
backends differ in is three operations on the key -> bytes store below:
_publish (shm: tmp + fsync + rename; tcp: push to the relay), _fetch (shm:
read the file; tcp: take from the relay, which hands a blob out once) and
_discard (shm: unlink; tcp: nothing is left to remove).
"""
import collections
import os
import pickle
import tempfile
import threading
import time
import uuid
from dataclasses import dataclass

import numpy as np

from .connector import tcp as _tcp
from .connector import transport as _kv
from .connector import wire as _wire
from .paths import SHM_ROOT
from .rm_compat import (ContractError, KVLayout, Measurement, MemoryTier,  # noqa: F401
                        TransferHandle, TransferPlan, TransferResult, TransportError)

COMPONENT = "rngd-pd"
WIRE_DTYPES = ("bf16", "fp16")          # 2-byte element types the wire carries
MEASUREMENT = "kv_transfer_ms"


@dataclass
class _Transfer:
    plan: object
    key: str
    t0: float
    kv: object = None                   # the decoded float32 array once landed


class _Ledger:
    """Transfers of one adapter, by handle token while in flight and by
    (request id, token range) once landed."""

    def __init__(self):
        self._lock = threading.Lock()
        self._in_flight = {}
        self._landed = {}

    def open(self, token, transfer):
        with self._lock:
            self._in_flight[token] = transfer

    def close_wait(self, token):
        with self._lock:
            return self._in_flight.pop(token, None)

    def land(self, transfer):
        with self._lock:
            self._landed[(transfer.plan.request_id, tuple(transfer.plan.tokens))] = transfer

    def claim(self, plan):
        with self._lock:
            return self._landed.pop((plan.request_id, tuple(plan.tokens)), None)

    def drain(self):
        """Every transfer still held (in flight or landed), forgetting them."""
        with self._lock:
            held = list(self._in_flight.values()) + list(self._landed.values())
            self._in_flight.clear()
            self._landed.clear()
        return held


def _refusal(t, src, dst, src_layout, dst_layout, tokens):
    """Why ``t`` cannot plan this transfer, or None."""
    if not t.supports(src, dst):
        return (f"{t.name} moves KV {t.SCOPE}; cannot plan "
                f"{src.name} ({src.kind}) to {dst.name} ({dst.kind})")
    src_layout.validate()
    dst_layout.validate()
    if src_layout != dst_layout:
        return (f"{t.name} does not convert layouts ({src_layout} vs {dst_layout}); "
                f"the model adapter must")
    if src_layout.dtype not in WIRE_DTYPES:
        return f"{t.name} carries 2-byte {'/'.join(WIRE_DTYPES)} values, not {src_layout.dtype}"
    start, end = tokens
    if start < 0 or end <= start:
        return f"{t.name}: token range {tuple(tokens)} is empty or negative"
    return None


class _TierTransfers:
    """The rm-core KVTransport methods, over a backend's _publish / _fetch /
    _discard. A subclass sets ``name`` and ``SCOPE`` and supplies supports()
    and _route() (what plan() puts in ``detail`` besides the wire dtype)."""

    def _start_ledger(self):
        self._ledger = _Ledger()
        self.measurements = collections.deque(maxlen=1024)

    def plan(self, request_id, src, dst, src_layout, dst_layout, tokens):
        why = _refusal(self, src, dst, src_layout, dst_layout, tokens)
        if why:
            raise TransportError(why)
        start, end = tokens
        detail = dict(self._route())
        detail["wire"] = src_layout.dtype
        return TransferPlan(request_id, src.validate(), dst.validate(), src_layout, dst_layout,
                            (start, end), (end - start) * src_layout.bytes_per_token(),
                            detail=detail)

    def submit(self, plan, kv=None):
        """kv: the range's KV, nbytes / 2 elements in any shape; zeros if omitted."""
        count = plan.nbytes // 2
        arr = np.zeros(count, np.float32) if kv is None else np.asarray(kv, np.float32)
        if arr.size != count:
            raise ContractError(f"{self.name}: plan {plan.request_id} {plan.tokens} moves "
                                f"{count} elements, kv holds {arr.size}")
        token = uuid.uuid4().hex
        key = "%s/%s/%d-%d.%s" % (plan.request_id, plan.dst.name, plan.tokens[0],
                                  plan.tokens[1], token[:8])
        transfer = _Transfer(plan, key, time.perf_counter())
        self._publish(key, _wire.ser(arr, plan.detail.get("wire", "bf16")))
        self._ledger.open(token, transfer)
        return TransferHandle(plan.request_id, self.name, token)

    def wait(self, handle, timeout_s):
        transfer = self._ledger.close_wait(handle.token)
        if transfer is None:
            raise TransportError(f"{self.name}: handle {handle.token} was never submitted here "
                                 f"or has been waited already")
        plan = transfer.plan
        try:
            kv = _wire.deser(self._fetch(transfer.key, timeout_s))
            error = None
            if kv.size * 2 != plan.nbytes:
                error = f"short segment: {kv.size * 2} of the {plan.nbytes} bytes the plan moved"
        except TimeoutError as e:
            kv, error = None, f"segment never arrived: {e}"
        except (ValueError, EOFError, OSError, pickle.UnpicklingError) as e:   # not a blob
            kv, error = None, f"segment unreadable: {e}"
        seconds = time.perf_counter() - transfer.t0
        if error:
            self._discard(transfer.key)
            got = 0 if kv is None else kv.size * 2
            return TransferResult(plan.request_id, False, got, seconds, error)
        transfer.kv = kv
        self._ledger.land(transfer)
        self.measurements.append(Measurement(
            MEASUREMENT, seconds * 1e3, {"component": COMPONENT, "kv_transport": self.name}
        ).validate())
        return TransferResult(plan.request_id, True, plan.nbytes, seconds)

    def take(self, plan):
        """The landed KV of ``plan`` (float32, the shape submit() was given); consumed."""
        transfer = self._ledger.claim(plan)
        if transfer is None:
            raise TransportError(f"{self.name}: no landed transfer for {plan.request_id} "
                                 f"tokens {tuple(plan.tokens)}")
        self._discard(transfer.key)
        return transfer.kv

    def _forget_all(self):
        for transfer in self._ledger.drain():
            self._discard(transfer.key)


def _two_host_tiers(prefix):
    return (MemoryTier(f"{prefix}-prefill", "host-dram", 1 << 30),
            MemoryTier(f"{prefix}-decode", "host-dram", 1 << 30),
            KVLayout(num_layers=2, num_kv_heads=2, head_dim=8, dtype="bf16"))


class ShmTransport(_TierTransfers, _kv.ShmTransport):
    """KV between two host-memory tiers of one machine, through /dev/shm files.

    root: the shared directory, default $PD_SHM_ROOT, else the serving root
    (/dev/shm/rngd_kv_cluster). Constructing one creates nothing; the directory
    appears with the first publish. A published segment is complete before
    its name exists (tmp + fsync + rename), so wait() never sees half a blob."""

    name = "shm"
    SCOPE = "only host-dram -> host-dram on one machine"

    def __init__(self, root=None):
        self.root = str(root or os.environ.get("PD_SHM_ROOT") or SHM_ROOT)
        self._private_dir = None
        self._start_ledger()

    def push(self, key, buf):
        self.push_parts(key, [buf])

    def push_parts(self, key, parts):
        os.makedirs(self.root, exist_ok=True)
        super().push_parts(key, parts)

    def supports(self, src, dst):
        return src.kind == dst.kind == "host-dram" and src.name != dst.name

    def _route(self):
        return {"root": self.root}

    def _publish(self, key, blob):
        self.push(key, blob)

    def _fetch(self, key, timeout):
        return self.pull(key, timeout=timeout)

    def _discard(self, key):
        self.discard(key)

    def close(self):
        """Discard every segment this instance published that was not taken,
        and the private conformance directory if it made one."""
        self._forget_all()
        if self._private_dir:
            try:
                os.rmdir(self._private_dir)
            except OSError:
                pass                     # someone else's files are in it: leave them
            self._private_dir = None

    def conformance_case(self):
        """Two host tiers sharing /dev/shm, in a private directory beside the
        serving root (rngd_kv_conformance.<uid>.<pid>), so a check never writes
        where live workers read. NoHardware if it cannot be written."""
        from .rm_compat import NoHardware
        parent = os.path.dirname(self.root.rstrip("/")) or "/dev/shm"
        private = os.path.join(parent, f"rngd_kv_conformance.{os.getuid()}.{os.getpid()}")
        try:
            os.makedirs(private, exist_ok=True)
            tempfile.TemporaryFile(dir=private).close()
        except OSError as e:
            raise NoHardware(f"cannot write a conformance directory at {private}: {e}") from e
        self.root = self._private_dir = private
        return _two_host_tiers("shm")


class TcpTransport(_TierTransfers, _tcp.TcpTransport):
    """KV between two host-memory tiers of any two machines, through one relay
    (the native librngdpd_net.so; the reference's airm.py:224-271).

    remote: (host, port) of the relay both sides use (default $AIRM_KV_TCP_ADDR);
    serve_port: also run a relay in this process. Every blob carries a CRC-32
    that the relay and the receiver check, so a good wait() has the bytes
    submit() sent. The relay hands a blob out once; the landed transfer keeps
    it for take()."""

    name = "tcp"
    SCOPE = "only host-dram -> host-dram"

    def __init__(self, remote=None, serve_port=None):
        _tcp.TcpTransport.__init__(self, remote=remote, serve_port=serve_port)
        self._start_ledger()

    def supports(self, src, dst):
        return src.kind == dst.kind == "host-dram" and src.name != dst.name

    def _route(self):
        return {"server": "%s:%d" % self.remote if self.remote else None}

    def _publish(self, key, blob):
        self.push(key, blob)

    def _fetch(self, key, timeout):
        return self.pull(key, timeout=timeout)

    def _discard(self, key):
        pass                             # the relay gave the blob away when it was fetched

    def close(self):
        self._forget_all()
        _tcp.TcpTransport.close(self)

    def conformance_case(self):
        """Two host tiers and a relay on a free loopback port in this process."""
        if self.remote is None:
            _tcp.TcpTransport.__init__(self, serve_port=0)
        return _two_host_tiers("tcp")
