"""The rm-core v0.1.1 surface this package's ``airm`` adapter uses.

When ``rm_core`` is importable its own classes are re-exported unchanged. When
it is not (it is a git dependency, ai-computing/rm-core@v0.1.1, that needs the
network to install), a local stand-in provides the same names with the
behaviour the reference's call sites rely on:

  KVLayout(num_layers, num_kv_heads, head_dim, dtype)   airm.py:221, tests/test_airm.py:183
      bytes_per_token() = 2 * layers * heads * head_dim * dtype bytes
      (consistent with connector/transport.py:257, "2 B/token" for 1x1x1 int8)
  MemoryTier(name, kind, capacity_bytes, locator="")    airm.py:219-220, tests/test_airm.py:181
  TransferPlan(request_id, src, dst, src_layout, dst_layout, tokens, nbytes, detail)
                                                         airm.py:86-88
  TransferHandle(request_id, transport, token)          airm.py:105
  TransferResult(request_id, ok, nbytes, seconds, error="")   airm.py:116-126
  Measurement(name, value, tags).validate()             airm.py:121-123
  ContractError, TransportError, conformance.NoHardware

The stand-in is a test double for the contract: rm-core's own conformance
checks (``rm_core.conformance.check_kv_transport``) are not reproduced bit for
bit; ``check_kv_transport`` here runs the plan/submit/wait/take/close sequence
the adapter's ``conformance_case`` is built for (airm.py:204-221).
"""
import collections
import importlib
import time
from dataclasses import dataclass, field

try:  # pragma: no cover - exercised only where rm-core is installed
    import rm_core as _rm
    from rm_core import (ContractError, KVLayout, Measurement, MemoryTier, TransferHandle,  # noqa: F401
                         TransferPlan, TransferResult, TransportError, prometheus_name)
    from rm_core.conformance import NoHardware, check_kv_transport  # noqa: F401
    from rm_core import registry  # noqa: F401
    HAVE_RM_CORE = True
except ImportError:
    _rm = None
    HAVE_RM_CORE = False

if not HAVE_RM_CORE:
    _DTYPE_BYTES = {"bf16": 2, "fp16": 2, "fp32": 4, "fp8": 1, "int8": 1}
    _TIER_KINDS = ("host-dram", "device-hbm", "device-dram", "cxl", "nvme")

    class ContractError(ValueError):
        """A value breaks the rm-core data contract."""

    class TransportError(RuntimeError):
        """A transport refuses or fails a transfer."""

    class NoHardware(RuntimeError):
        """The environment cannot host a conformance case."""

    @dataclass(frozen=True)
    class KVLayout:
        num_layers: int
        num_kv_heads: int
        head_dim: int
        dtype: str

        def bytes_per_token(self):
            return 2 * self.num_layers * self.num_kv_heads * self.head_dim * _DTYPE_BYTES[self.dtype]

        def validate(self):
            if min(self.num_layers, self.num_kv_heads, self.head_dim) <= 0:
                raise ContractError(f"layout dimensions must be positive: {self}")
            if self.dtype not in _DTYPE_BYTES:
                raise ContractError(f"unknown dtype {self.dtype!r}")
            return self

    @dataclass(frozen=True)
    class MemoryTier:
        name: str
        kind: str
        capacity_bytes: int
        locator: str = ""

        def validate(self):
            if not self.name:
                raise ContractError("tier needs a name")
            if self.kind not in _TIER_KINDS:
                raise ContractError(f"unknown tier kind {self.kind!r}")
            if self.capacity_bytes <= 0:
                raise ContractError("tier capacity must be positive")
            return self

    @dataclass
    class TransferPlan:
        request_id: str
        src: MemoryTier
        dst: MemoryTier
        src_layout: KVLayout
        dst_layout: KVLayout
        tokens: tuple
        nbytes: int
        detail: dict = field(default_factory=dict)

    @dataclass(frozen=True)
    class TransferHandle:
        request_id: str
        transport: str
        token: str

    @dataclass
    class TransferResult:
        request_id: str
        ok: bool
        nbytes: int
        seconds: float
        error: str = ""

    @dataclass
    class Measurement:
        name: str
        value: float
        tags: dict = field(default_factory=dict)

        def validate(self):
            if not self.name or not isinstance(self.value, (int, float)):
                raise ContractError(f"bad measurement {self!r}")
            return self

    def prometheus_name(name):
        return "airm_" + name

    class _Registry:
        """Entry-point registry over this package's own ``airm.kv_transports``."""

        GROUPS = {"airm.kv_transports": {"shm": "rngd_pd_amd.airm:ShmTransport"}}

        def available(self, group):
            return dict(self.GROUPS.get(group, {}))

        def load(self, group, name, **kw):
            target = self.GROUPS.get(group, {}).get(name)
            if target is None:
                raise KeyError(f"{group}: no entry point named {name!r}")
            mod, obj = target.split(":")
            return getattr(importlib.import_module(mod), obj)(**kw)

    registry = _Registry()

    def check_kv_transport(t, timeout_s=5.0):
        """plan -> submit -> wait -> take -> close on the transport's own case,
        checking the bf16 round trip and the refusal of a bad token range."""
        import numpy as np
        src, dst, layout = t.conformance_case()
        try:
            try:
                t.plan("conf-bad", src, dst, layout, layout, (4, 4))
            except TransportError:
                pass
            else:
                raise AssertionError("empty token range was not refused")
            plan = t.plan("conf", src, dst, layout, layout, (0, 4))
            n = plan.nbytes // 2
            kv = np.random.default_rng(7).standard_normal(n).astype(np.float32)
            res = t.wait(t.submit(plan, kv=kv), timeout_s=timeout_s)
            if not res.ok or res.nbytes != plan.nbytes:
                raise AssertionError(f"transfer failed: {res}")
            got = np.asarray(t.take(plan), np.float32).reshape(-1)
            want = (kv.view(np.uint32) >> 16 << 16).view(np.float32)
            if plan.detail.get("wire", "bf16") == "bf16" and not np.array_equal(
                    got.view(np.uint32), want.view(np.uint32)):
                raise AssertionError("payload changed in transit")
            if not t.measurements or t.measurements[-1].name != "kv_transfer_ms":
                raise AssertionError("no kv_transfer_ms measurement recorded")
        finally:
            t.close()

    class LoopbackTransport:
        """Tier-to-tier transport that completes at once (a test double for the
        ``FencedTransport`` path; rm-core ships one as rm_core.reference)."""

        name = "loopback"

        def __init__(self, fail_request_ids=()):
            self.fail = set(fail_request_ids)
            self._handles = {}
            self.measurements = collections.deque(maxlen=1024)

        def plan(self, request_id, src, dst, src_layout, dst_layout, tokens):
            start, end = tokens
            if not 0 <= start < end:
                raise TransportError(f"bad token range {tokens}")
            return TransferPlan(request_id, src, dst, src_layout, dst_layout, tokens,
                                (end - start) * src_layout.bytes_per_token())

        def submit(self, plan, kv=None):
            token = f"{len(self._handles)}.{time.perf_counter_ns()}"
            self._handles[token] = plan
            return TransferHandle(plan.request_id, self.name, token)

        def wait(self, handle, timeout_s):
            plan = self._handles.pop(handle.token, None)
            if plan is None:
                raise TransportError(f"unknown handle {handle.token}")
            if plan.request_id in self.fail:
                return TransferResult(plan.request_id, False, 0, 0.0, "injected failure")
            return TransferResult(plan.request_id, True, plan.nbytes, 0.0)

        def close(self):
            self._handles.clear()

    registry.GROUPS["airm.kv_transports"]["loopback"] = "rngd_pd_amd.rm_compat:LoopbackTransport"
