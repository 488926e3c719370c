"""Test doubles for the parts of rm-core v0.1.1 this package meets but does not ship.

rm-core is a git dependency that is absent offline, so the tests stand in for:

  LoopbackTransport   a tier-to-tier KVTransport that completes at once (rm-core
                      ships one as rm_core.reference.LoopbackTransport; the
                      reference's tests select it by name, tests/test_airm.py:105-116)
  RegistryDouble      an ``airm.kv_transports`` entry-point registry holding
                      chosen names, installed as rm_compat.registry for a test
  check_kv_transport  the plan -> submit -> wait -> take -> close sequence a
                      conformance case is built for (airm.py:204-221): the
                      refusal of an empty range, the bf16 round trip and the
                      kv_transfer_ms measurement. rm-core's own checks are not
                      reproduced (parity unpinned).
"""
import importlib
import itertools

import numpy as np

from rngd_pd_amd.rm_compat import TransferHandle, TransferPlan, TransferResult, TransportError


class LoopbackTransport:
    """Completes every transfer at submit(); request ids in ``fail_request_ids`` fail."""

    name = "loopback"

    def __init__(self, fail_request_ids=()):
        self.fail = set(fail_request_ids)
        self._handles = {}
        self._ids = itertools.count()

    def plan(self, request_id, src, dst, src_layout, dst_layout, tokens):
        start, end = tokens
        if start < 0 or end <= start:
            raise TransportError(f"loopback: empty range {tokens}")
        return TransferPlan(request_id, src, dst, src_layout, dst_layout, tokens,
                            (end - start) * src_layout.bytes_per_token())

    def submit(self, plan, kv=None):
        token = f"lb{next(self._ids)}"
        self._handles[token] = plan
        return TransferHandle(plan.request_id, self.name, token)

    def wait(self, handle, timeout_s):
        plan = self._handles.pop(handle.token, None)
        if plan is None:
            raise TransportError(f"loopback: no handle {handle.token}")
        if plan.request_id in self.fail:
            return TransferResult(plan.request_id, False, 0, 0.0, "failure injected by the test")
        return TransferResult(plan.request_id, True, plan.nbytes, 0.0)

    def close(self):
        self._handles.clear()


class RegistryDouble:
    """``group -> {name: "module:attr"}`` with rm-core's registry methods."""

    def __init__(self, groups):
        self.groups = {g: dict(m) for g, m in groups.items()}
        self.loads = 0

    def available(self, group):
        return dict(self.groups.get(group, {}))

    def load(self, group, name, **kw):
        target = self.groups.get(group, {}).get(name)
        if target is None:
            raise KeyError(f"{group}: no entry point {name!r}")
        self.loads += 1
        module, attr = target.split(":")
        return getattr(importlib.import_module(module), attr)(**kw)


def check_kv_transport(t, timeout_s=5.0):
    src, dst, layout = t.conformance_case()
    try:
        try:
            t.plan("conformance-empty", src, dst, layout, layout, (3, 3))
        except TransportError:
            pass
        else:
            raise AssertionError("an empty token range was planned")
        plan = t.plan("conformance", src, dst, layout, layout, (0, 4))
        kv = np.random.default_rng(7).standard_normal(plan.nbytes // 2).astype(np.float32)
        res = t.wait(t.submit(plan, kv=kv), timeout_s=timeout_s)
        if not res.ok or res.nbytes != plan.nbytes:
            raise AssertionError(f"transfer failed: {res}")
        got = np.asarray(t.take(plan), np.float32).reshape(-1)
        if plan.detail.get("wire", "bf16") == "bf16":
            want = (kv.view(np.uint32) >> 16 << 16).view(np.float32)
            if not np.array_equal(got.view(np.uint32), want.view(np.uint32)):
                raise AssertionError("the payload changed in transit")
        if not t.measurements or t.measurements[-1].name != "kv_transfer_ms":
            raise AssertionError("no kv_transfer_ms measurement was recorded")
    finally:
        t.close()
