"""Transport selection and the rm-core ``shm`` adapter.

Restates the reference's tests/test_airm.py (SelectionTests, ShmTransportTests,
test_constructing_does_not_create_root) against this package. rm-core itself
is not installed here, so the checks run against rngd_pd_amd.rm_compat's
stand-in (its conformance runner and loopback transport are test doubles).
"""
import os
import sys
import tempfile
import unittest
from unittest import mock

import numpy as np

from oracle import wire as owire
from rngd_pd_amd import airm, rm_compat
from rngd_pd_amd.connector import transport as kv

NL, NKV, S, HD = 4, 8, 16, 128


def _kv(seed):
    rng = np.random.default_rng(seed)
    return ([rng.standard_normal((NKV, S, HD)).astype(np.float32) for _ in range(NL)],
            [rng.standard_normal((NKV, S, HD)).astype(np.float32) for _ in range(NL)])


def _handoff(prefill_transport, decode_transport, req_id="r1"):
    """prefill save -> transport -> decode load through the connector, bf16 wire."""
    from rngd_pd_amd.connector.rngd_kv import KVConnectorRole, RngdKVConnector
    ck, cv = _kv(0)
    pf = RngdKVConnector(KVConnectorRole.WORKER, req_id=req_id, transport=prefill_transport,
                         n_layers=NL)
    for i in range(NL):
        pf.save_kv_layer(f"layer.{i}", (ck[i], cv[i]))
    dk = [np.zeros((NKV, S, HD), np.float32) for _ in range(NL)]
    dv = [np.zeros((NKV, S, HD), np.float32) for _ in range(NL)]
    dc = RngdKVConnector(KVConnectorRole.WORKER, req_id=req_id, transport=decode_transport,
                         n_layers=NL)
    dc.register_kv_caches((dk, dv))
    dc.bind_connector_metadata(dc.build_connector_meta(None))
    dc.start_load_kv()
    for i in range(NL):
        dc.wait_for_layer_load(f"layer.{i}")
    return np.stack(dk), np.stack(dv)


class _Env:
    """A temporary shm root and the bf16 wire, restored afterwards."""

    def setUp(self):
        self.tmp = tempfile.TemporaryDirectory(dir="/dev/shm" if os.access("/dev/shm", os.W_OK) else None)
        self.wire = kv.WIRE
        kv.WIRE = "bf16"
        kv._FENCED.clear(); kv._CLASSES.clear(); kv._SHARED.clear()   # noqa: E702
        self.env = mock.patch.dict(os.environ, {"PD_SHM_ROOT": self.tmp.name})
        self.env.start()
        os.environ.pop("AIRM_KV_TRANSPORT", None)

    def tearDown(self):
        self.env.stop()
        kv.WIRE = self.wire
        kv._FENCED.clear(); kv._CLASSES.clear(); kv._SHARED.clear()   # noqa: E702
        self.tmp.cleanup()


class SelectionTests(_Env, unittest.TestCase):
    def test_shm_is_registered_and_default(self):
        self.assertEqual(rm_compat.registry.available("airm.kv_transports").get("shm"),
                         "rngd_pd_amd.airm:ShmTransport")
        t = kv.select_transport()
        self.assertIsInstance(t, airm.ShmTransport)
        self.assertIsInstance(t, kv.ShmTransport)
        self.assertEqual(t.root, self.tmp.name)

    def test_env_shm_same_output_as_before(self):
        """AIRM_KV_TRANSPORT=shm gives bit for bit the KV a hard-coded ShmTransport gives."""
        before = _handoff(kv.ShmTransport(self.tmp.name + "/legacy"),
                          kv.ShmTransport(self.tmp.name + "/legacy"))
        os.environ["AIRM_KV_TRANSPORT"] = "shm"
        after = _handoff(None, None, req_id="r2")
        for a, b in zip(before, after):
            np.testing.assert_array_equal(a.view(np.uint32), b.view(np.uint32))
        self.assertTrue(np.any(after[0]))

    def test_handoff_equals_bf16_truncation(self):
        os.environ["AIRM_KV_TRANSPORT"] = "shm"
        dk, dv = _handoff(None, None, req_id="r4")
        ck, cv = _kv(0)
        ref = lambda a: (a.view(np.uint32) >> 16 << 16).view(np.float32)   # noqa: E731
        np.testing.assert_array_equal(dk, ref(np.stack(ck)))
        np.testing.assert_array_equal(dv, ref(np.stack(cv)))

    def test_files_match_reference_protocol(self):
        """The connector's files are the oracle's restatement of the reference's files."""
        t = kv.ShmTransport(self.tmp.name + "/a")
        _handoff(t, t, req_id="rq")
        ck, cv = _kv(0)
        for i in range(NL):
            for which, arr in (("k", ck[i]), ("v", cv[i])):
                with open(os.path.join(t.root, f"rq__layer.{i}__{which}"), "rb") as f:
                    self.assertEqual(f.read(), owire.ser(arr, "bf16"))

    def test_old_and_new_shm_interoperate(self):
        """The oracle's file protocol and this transport read each other's files."""
        new = kv.select_transport("shm")
        owire.shm_push(self.tmp.name, "req/layer.0/k", b"abc")
        self.assertEqual(new.pull("req/layer.0/k", timeout=1), b"abc")
        new.push("req/layer.0/v", b"xyz")
        self.assertEqual(owire.shm_pull(self.tmp.name, "req/layer.0/v", timeout=1), b"xyz")

    def test_push_parts_and_pull_into(self):
        t = kv.ShmTransport(self.tmp.name)
        t.push_parts("a/b", [b"he", memoryview(b"llo "), bytearray(b"world")])
        self.assertEqual(t.pull("a/b"), b"hello world")
        buf = bytearray(32)
        self.assertEqual(t.pull_into("a/b", buf), 11)
        self.assertEqual(bytes(buf[:11]), b"hello world")
        self.assertEqual(t.pull_size("a/b"), 11)
        with self.assertRaises(ValueError):
            t.pull_into("a/b", bytearray(4))
        self.assertFalse([f for f in os.listdir(self.tmp.name) if ".tmp." in f])

    def test_pull_timeout(self):
        t = kv.select_transport("shm")
        with self.assertRaises(TimeoutError):
            t.pull("nope/layer.0/k", timeout=0.01)

    def test_config_alone_selects_another_name(self):
        os.environ["AIRM_KV_TRANSPORT"] = "loopback"        # a tier-to-tier test double
        from rngd_pd_amd.connector.rngd_kv import KVConnectorRole, RngdKVConnector
        conn = RngdKVConnector(KVConnectorRole.WORKER, req_id="r", n_layers=NL)
        self.assertIsInstance(conn.t, kv.FencedTransport)
        self.assertIsInstance(conn.t.impl, rm_compat.LoopbackTransport)
        dk, dv = _handoff(None, None, req_id="r3")
        ck, cv = _kv(0)
        ref = lambda a: (a.view(np.uint32) >> 16 << 16).view(np.float32)   # noqa: E731
        np.testing.assert_array_equal(dk, ref(np.stack(ck)))
        np.testing.assert_array_equal(dv, ref(np.stack(cv)))

    def test_unknown_name_fails_loud(self):
        os.environ["AIRM_KV_TRANSPORT"] = "no-such-path"
        with self.assertRaises(KeyError):
            kv.select_transport()
        with self.assertRaises(KeyError):
            kv.select_transport("nixl-ucx")           # a vendor P2P path this package lacks

    def test_shm_without_rm_core(self):
        with mock.patch.dict(sys.modules, {"rm_core": None}):
            t = kv.select_transport("shm")
            self.assertIsInstance(t, kv.ShmTransport)
            self.assertEqual(t.root, self.tmp.name)
            with self.assertRaises(KeyError):
                kv.select_transport("p2p")

    def test_class_resolved_once(self):
        kv.select_transport("shm")
        with mock.patch.object(rm_compat.registry, "load", side_effect=AssertionError("rescanned")):
            self.assertIsInstance(kv.select_transport("shm"), airm.ShmTransport)

    def test_fenced_duplicate_push_and_close(self):
        t = kv.select_transport("loopback")
        t.push("k", b"ab")
        with self.assertRaises(ValueError):
            t.push("k", b"cd")
        self.assertEqual(t.pull("k", timeout=1), b"ab")
        t.close()
        self.assertIsNot(kv.select_transport("loopback"), t)

    def test_fenced_failure_raises(self):
        t = kv.FencedTransport(rm_compat.LoopbackTransport(fail_request_ids=["req/layer.0/k"]))
        t.push("req/layer.0/k", b"abcd")
        with self.assertRaises(rm_compat.TransportError):
            t.pull("req/layer.0/k", timeout=1)

    def test_make_transport(self):
        self.assertIsInstance(kv.make_transport("inproc"), kv.InProcTransport)
        with self.assertRaises(NotImplementedError):
            kv.make_transport("nixl")
        with self.assertRaises(NotImplementedError):
            kv.make_transport("nixl-ucx")
        from rngd_pd_amd.connector.tcp import TcpTransport
        self.assertIsInstance(kv.make_transport("tcp"), TcpTransport)
        with self.assertRaises(ValueError):
            kv.make_transport("carrier-pigeon")


class ShmAdapterTests(_Env, unittest.TestCase):
    def test_conformance(self):
        t = airm.ShmTransport()
        rm_compat.check_kv_transport(t)
        self.assertEqual(os.listdir(self.tmp.name), [])     # it used its own directory
        self.assertTrue(t.measurements)
        self.assertEqual(t.measurements[-1].tags["kv_transport"], "shm")

    def test_payload_round_trip(self):
        t = airm.ShmTransport()
        src, dst, layout = t.conformance_case()
        kv_in = np.random.default_rng(1).standard_normal((2, 2, 4, 2, 8)).astype(np.float32)
        plan = t.plan("q", src, dst, layout, layout, (0, 4))
        self.assertEqual(plan.nbytes, 4 * 2 * 2 * 2 * 8 * 2)
        self.assertEqual(plan.detail, {"root": t.root, "wire": "bf16"})
        res = t.wait(t.submit(plan, kv=kv_in), timeout_s=5)
        self.assertTrue(res.ok)
        got = t.take(plan).reshape(kv_in.shape)
        np.testing.assert_array_equal(got.view(np.uint32), kv_in.view(np.uint32) >> 16 << 16)
        with self.assertRaises(rm_compat.TransportError):
            t.take(plan)                                     # consumed
        t.close()

    def test_rejects_unsupported(self):
        t = airm.ShmTransport()
        src, dst, layout = t.conformance_case()
        dev = rm_compat.MemoryTier("gpu0", "device-hbm", 1 << 30, "n/mi355x:0")
        for args in [(dev, dst, layout, layout, (0, 4)),
                     (src, dst, layout, rm_compat.KVLayout(2, 2, 16, "bf16"), (0, 4)),
                     (src, dst, rm_compat.KVLayout(2, 2, 8, "fp8"),
                      rm_compat.KVLayout(2, 2, 8, "fp8"), (0, 4)),
                     (src, dst, layout, layout, (4, 4))]:
            with self.assertRaises(rm_compat.TransportError):
                t.plan("bad", *args)
        t.close()

    def test_wait_reports_missing_and_short_segments(self):
        t = airm.ShmTransport()
        src, dst, layout = t.conformance_case()
        plan = t.plan("m", src, dst, layout, layout, (0, 4))
        h = t.submit(plan)
        key = next(iter(t._written))
        os.unlink(t._path(key))
        res = t.wait(h, timeout_s=0.05)
        self.assertFalse(res.ok)
        with self.assertRaises(rm_compat.TransportError):
            t.wait(h, timeout_s=0.05)                       # already waited
        before = set(t._written)
        h2 = t.submit(plan)
        (key2,) = set(t._written) - before
        with open(t._path(key2), "wb") as f:
            f.write(owire.ser(np.zeros(3, np.float32), "bf16"))
        res = t.wait(h2, timeout_s=1)
        self.assertFalse(res.ok)
        self.assertIn("plan moved", res.error)
        with self.assertRaises(rm_compat.ContractError):
            t.submit(plan, kv=np.zeros(5, np.float32))
        t.close()

    def test_close_removes_own_keys_only(self):
        t = airm.ShmTransport()
        src, dst, layout = t.conformance_case()
        other = os.path.join(t.root, "someone__else")
        open(other, "wb").close()
        plan = t.plan("c", src, dst, layout, layout, (0, 2))
        t.submit(plan)
        t.close()
        self.assertEqual(os.listdir(t.root), ["someone__else"])
        os.unlink(other)
        os.rmdir(t.root)


class ConstructionTests(unittest.TestCase):
    def test_constructing_does_not_create_root(self):
        with tempfile.TemporaryDirectory() as d:
            root = os.path.join(d, "never")
            airm.ShmTransport(root=root)
            self.assertFalse(os.path.exists(root))

    def test_layout_bytes_per_token(self):
        self.assertEqual(rm_compat.KVLayout(1, 1, 1, "int8").bytes_per_token(), 2)
        self.assertEqual(rm_compat.KVLayout(32, 8, 128, "bf16").bytes_per_token(), 131072)
