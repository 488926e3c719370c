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

Without rm-core there is no ``registry`` (None): transport selection then
knows only this package's own transports, as the reference's does
(connector/transport.py:307-318). rm-core's conformance runner
(``rm_core.conformance.check_kv_transport``) and its reference transports are
not part of this package; the tests carry doubles of them.
"""
from dataclasses import dataclass, field

try:  # pragma: no cover - exercised only where rm-core is installed
    import rm_core as _rm
    from rm_core import (ContractError, KVLayout, Measurement, MemoryTier, TransferHandle,  # noqa: F401
                         TransferPlan, TransferResult, TransportError, prometheus_name)
    from rm_core.conformance import NoHardware  # noqa: F401
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

    # Without rm-core there is no entry-point registry: select_transport then
    # resolves only this package's own transports (shm, tcp, ipc).
    registry = None
