"""Transport selection, the connector's host path over it, and the rm-core adapter.

The cases restate the reference's tests/test_airm.py against this package with
its vectors: seed 0 layers of [8, 16, 128] (4 layers, K then V) through the
connector, seed 1 KV of shape (2, 2, 4, 2, 8) through the adapter, the bf16
truncation identity, raw-byte interop, and the refusals. rm-core is absent, so
its registry, reference transport and conformance runner are the doubles in
tests/rm_doubles.py.
"""
import os
import threading
import time

import numpy as np
import pytest

from oracle import wire as owire
from rngd_pd_amd import airm, rm_compat
from rngd_pd_amd.connector import transport as kv
from tests.rm_doubles import LoopbackTransport, RegistryDouble, check_kv_transport

NL, NKV, S, HD = 4, 8, 16, 128
GROUP = "airm.kv_transports"


def layers(seed):
    """K and V, each [NL, NKV, S, HD] float32 (the same draws as the reference's _kv(seed))."""
    both = np.random.default_rng(seed).standard_normal((2, NL, NKV, S, HD)).astype(np.float32)
    return both[0], both[1]


def truncated(a):
    return (a.view(np.uint32) >> 16 << 16).view(np.float32)


def connector_round_trip(save_t, load_t, req_id):
    """Save every layer of layers(0) through one connector and load it through another."""
    from rngd_pd_amd.connector.rngd_kv import KVConnectorRole, RngdKVConnector
    K, V = layers(0)
    producer = RngdKVConnector(KVConnectorRole.WORKER, req_id=req_id, transport=save_t,
                               n_layers=NL)
    for i in range(NL):
        producer.save_kv_layer(f"layer.{i}", (K[i], V[i]))
    gotK, gotV = np.zeros_like(K), np.zeros_like(V)
    consumer = RngdKVConnector(KVConnectorRole.WORKER, req_id=req_id, transport=load_t,
                               n_layers=NL)
    consumer.register_kv_caches((list(gotK), list(gotV)))
    consumer.bind_connector_metadata(consumer.build_connector_meta(None))
    consumer.start_load_kv()
    for i in range(NL):
        consumer.wait_for_layer_load(f"layer.{i}")
    return gotK, gotV


@pytest.fixture
def shm_root(tmp_path_factory, monkeypatch):
    """A private shm root as $PD_SHM_ROOT, the bf16 wire, and a clean selection."""
    base = "/dev/shm" if os.access("/dev/shm", os.W_OK) else None
    import tempfile
    root = tempfile.mkdtemp(prefix="pdk_transport_test.", dir=base)
    monkeypatch.setenv("PD_SHM_ROOT", root)
    monkeypatch.delenv("AIRM_KV_TRANSPORT", raising=False)
    monkeypatch.setattr(kv, "WIRE", "bf16")
    kv.reset_selection()
    yield root
    kv.reset_selection()
    import shutil
    shutil.rmtree(root, ignore_errors=True)


@pytest.fixture
def registry(monkeypatch):
    """An rm-core registry with this package's shm entry point and the loopback double."""
    reg = RegistryDouble({GROUP: {"shm": "rngd_pd_amd.airm:ShmTransport",
                                  "loopback": "tests.rm_doubles:LoopbackTransport"}})
    monkeypatch.setattr(rm_compat, "registry", reg)
    return reg


# -- selection -----------------------------------------------------------------

def test_default_is_the_shm_adapter(shm_root):
    t = kv.select_transport()
    assert isinstance(t, airm.ShmTransport) and isinstance(t, kv.ShmTransport)
    assert t.root == shm_root


def test_entry_points_declared():
    import tomli
    here = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    with open(os.path.join(here, "pyproject.toml"), "rb") as f:
        eps = tomli.load(f)["project"]["entry-points"][GROUP]
    assert eps["shm"] == "rngd_pd_amd.airm:ShmTransport"
    assert eps["tcp"] == "rngd_pd_amd.airm:TcpTransport"
    assert eps["ipc"] == "rngd_pd_amd.connector.ipc:IpcTransport"


def test_selected_shm_gives_the_same_kv_as_a_fixed_transport(shm_root, monkeypatch):
    fixed = kv.ShmTransport(os.path.join(shm_root, "fixed"))
    before = connector_round_trip(fixed, fixed, "r1")
    monkeypatch.setenv("AIRM_KV_TRANSPORT", "shm")
    after = connector_round_trip(None, None, "r2")
    for a, b in zip(before, after):
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    assert np.any(after[0])


def test_round_trip_is_bf16_truncation(shm_root, monkeypatch):
    monkeypatch.setenv("AIRM_KV_TRANSPORT", "shm")
    gotK, gotV = connector_round_trip(None, None, "r4")
    K, V = layers(0)
    assert np.array_equal(gotK, truncated(K)) and np.array_equal(gotV, truncated(V))


def test_files_are_the_reference_protocol(shm_root):
    t = kv.ShmTransport(os.path.join(shm_root, "a"))
    connector_round_trip(t, t, "rq")
    K, V = layers(0)
    for i in range(NL):
        for which, arr in (("k", K[i]), ("v", V[i])):
            with open(os.path.join(t.root, f"rq__layer.{i}__{which}"), "rb") as f:
                assert f.read() == owire.ser(arr, "bf16")


def test_raw_bytes_interoperate_with_the_oracle_protocol(shm_root):
    t = kv.select_transport("shm")
    owire.shm_push(shm_root, "req/layer.0/k", b"abc")
    assert t.pull("req/layer.0/k", timeout=1) == b"abc"
    t.push("req/layer.0/v", b"xyz")
    assert owire.shm_pull(shm_root, "req/layer.0/v", timeout=1) == b"xyz"


def test_push_parts_pull_into_and_discard(shm_root):
    t = kv.ShmTransport(shm_root)
    t.push_parts("a/b", [b"he", memoryview(b"llo "), bytearray(b"world")])
    assert t.pull("a/b") == b"hello world"
    buf = bytearray(32)
    assert t.pull_into("a/b", buf) == 11 and bytes(buf[:11]) == b"hello world"
    assert t.pull_size("a/b") == 11
    with pytest.raises(ValueError):
        t.pull_into("a/b", bytearray(4))
    assert not [f for f in os.listdir(shm_root) if ".tmp." in f]
    t.discard("a/b")
    t.discard("a/b")                                    # already gone: no error
    assert os.listdir(shm_root) == []


def test_discard_request_removes_only_that_request(shm_root):
    t = kv.ShmTransport(shm_root)
    for req in ("r1", "r10", "r1x"):
        for i in range(3):
            t.push(f"{req}/layer.{i}/k", b"k")
    assert t.discard_request("r1") == 3
    assert sorted(os.listdir(shm_root)) == sorted(
        [f"r10__layer.{i}__k" for i in range(3)] + [f"r1x__layer.{i}__k" for i in range(3)])


def test_pull_timeout(shm_root):
    with pytest.raises(TimeoutError):
        kv.select_transport("shm").pull("nope/layer.0/k", timeout=0.01)


def test_another_name_from_configuration_alone(shm_root, registry, monkeypatch):
    from rngd_pd_amd.connector.rngd_kv import KVConnectorRole, RngdKVConnector
    monkeypatch.setenv("AIRM_KV_TRANSPORT", "loopback")
    conn = RngdKVConnector(KVConnectorRole.WORKER, req_id="r", n_layers=NL)
    assert isinstance(conn.t, kv.FencedTransport) and isinstance(conn.t.impl, LoopbackTransport)
    gotK, gotV = connector_round_trip(None, None, "r3")
    K, V = layers(0)
    assert np.array_equal(gotK, truncated(K)) and np.array_equal(gotV, truncated(V))


def test_unknown_and_absent_names_raise(shm_root, registry):
    with pytest.raises(KeyError):
        kv.select_transport("no-such-path")
    with pytest.raises(KeyError):
        kv.select_transport("nixl-ucx")


def test_without_rm_core_only_own_transports_resolve(shm_root):
    assert rm_compat.registry is None                 # rm-core is not installed here
    t = kv.select_transport("shm")
    assert isinstance(t, kv.ShmTransport) and t.root == shm_root
    for name in ("p2p", "loopback"):
        with pytest.raises(KeyError):
            kv.select_transport(name)


def test_resolved_once_per_process(shm_root, registry):
    kv.select_transport("shm")
    kv.select_transport("shm")
    kv.select_transport("shm")
    assert registry.loads == 1


def test_fenced_duplicate_push_and_close(shm_root, registry):
    t = kv.select_transport("loopback")
    assert kv.select_transport("loopback") is t        # one per process: both ends share it
    t.push("k", b"ab")
    with pytest.raises(ValueError):
        t.push("k", b"cd")
    assert t.pull("k", timeout=1) == b"ab"
    t.close()
    assert kv.select_transport("loopback") is not t


def test_fenced_pull_waits_for_a_late_push():
    t = kv.FencedTransport(LoopbackTransport())
    threading.Timer(0.05, lambda: t.push("late", b"xy")).start()
    t0 = time.monotonic()
    assert t.pull("late", timeout=2) == b"xy"
    assert time.monotonic() - t0 >= 0.04
    with pytest.raises(TimeoutError):
        t.pull("never", timeout=0.02)


def test_fenced_failure_raises():
    t = kv.FencedTransport(LoopbackTransport(fail_request_ids=["req/layer.0/k"]))
    t.push("req/layer.0/k", b"abcd")
    with pytest.raises(rm_compat.TransportError):
        t.pull("req/layer.0/k", timeout=1)


def test_make_transport():
    assert isinstance(kv.make_transport("inproc"), kv.InProcTransport)
    for name in ("nixl", "nixl-ucx"):
        with pytest.raises(NotImplementedError):
            kv.make_transport(name)
    from rngd_pd_amd.connector.tcp import TcpTransport
    assert isinstance(kv.make_transport("tcp"), TcpTransport)
    with pytest.raises(ValueError):
        kv.make_transport("carrier-pigeon")


# -- the rm-core adapter -------------------------------------------------------

def test_adapter_conformance_sequence(shm_root):
    t = airm.ShmTransport()
    check_kv_transport(t)
    assert os.listdir(shm_root) == []                  # the check used its own directory
    assert t.measurements[-1].name == "kv_transfer_ms"
    assert t.measurements[-1].tags == {"component": "rngd-pd", "kv_transport": "shm"}


def test_adapter_payload_round_trip(shm_root):
    t = airm.ShmTransport()
    src, dst, layout = t.conformance_case()
    kv_in = np.random.default_rng(1).standard_normal((2, 2, 4, 2, 8)).astype(np.float32)
    plan = t.plan("q", src, dst, layout, layout, (0, 4))
    assert plan.nbytes == 4 * 2 * 2 * 2 * 8 * 2
    assert plan.detail == {"root": t.root, "wire": "bf16"}
    res = t.wait(t.submit(plan, kv=kv_in), timeout_s=5)
    assert res.ok and res.nbytes == plan.nbytes
    got = t.take(plan).reshape(kv_in.shape)
    assert np.array_equal(got.view(np.uint32), kv_in.view(np.uint32) >> 16 << 16)
    with pytest.raises(rm_compat.TransportError):
        t.take(plan)                                   # consumed
    assert os.listdir(t.root) == []                    # and its segment is gone
    t.close()


def test_adapter_refusals(shm_root):
    t = airm.ShmTransport()
    src, dst, layout = t.conformance_case()
    hbm = rm_compat.MemoryTier("gpu0", "device-hbm", 1 << 30, "n/mi355x:0")
    fp8 = rm_compat.KVLayout(2, 2, 8, "fp8")
    for args in [(hbm, dst, layout, layout, (0, 4)),
                 (src, dst, layout, rm_compat.KVLayout(2, 2, 16, "bf16"), (0, 4)),
                 (src, dst, fp8, fp8, (0, 4)),
                 (src, dst, layout, layout, (4, 4)),
                 (src, src, layout, layout, (0, 4))]:
        with pytest.raises(rm_compat.TransportError):
            t.plan("bad", *args)
    t.close()


def test_adapter_reports_missing_short_and_bad_segments(shm_root):
    t = airm.ShmTransport()
    src, dst, layout = t.conformance_case()
    plan = t.plan("m", src, dst, layout, layout, (0, 4))

    def submit_and_find():
        before = set(os.listdir(t.root))
        h = t.submit(plan)
        (name,) = set(os.listdir(t.root)) - before
        return h, os.path.join(t.root, name)

    h, path = submit_and_find()
    os.unlink(path)
    res = t.wait(h, timeout_s=0.05)
    assert not res.ok and res.nbytes == 0
    with pytest.raises(rm_compat.TransportError):
        t.wait(h, timeout_s=0.05)                      # already waited
    h, path = submit_and_find()
    with open(path, "wb") as f:
        f.write(owire.ser(np.zeros(3, np.float32), "bf16"))
    res = t.wait(h, timeout_s=1)
    assert not res.ok and res.nbytes == 6 and "plan moved" in res.error
    assert not os.path.exists(path)                    # a failed segment is discarded
    h, path = submit_and_find()
    with open(path, "wb") as f:
        f.write(b"not a pickle")
    res = t.wait(h, timeout_s=1)
    assert not res.ok and "unreadable" in res.error
    with pytest.raises(rm_compat.ContractError):
        t.submit(plan, kv=np.zeros(5, np.float32))
    t.close()


def test_adapter_close_removes_its_own_segments_only(shm_root):
    t = airm.ShmTransport()
    src, dst, layout = t.conformance_case()
    other = os.path.join(t.root, "someone__else")
    open(other, "wb").close()
    plan = t.plan("c", src, dst, layout, layout, (0, 2))
    t.submit(plan)                                     # in flight
    t.wait(t.submit(t.plan("d", src, dst, layout, layout, (0, 2))), timeout_s=1)   # landed
    t.close()
    assert os.listdir(t.root) == ["someone__else"]
    os.unlink(other)
    os.rmdir(t.root)


def test_constructing_does_not_create_the_root(tmp_path):
    root = tmp_path / "never"
    airm.ShmTransport(root=str(root))
    assert not root.exists()


def test_layout_bytes_per_token():
    assert rm_compat.KVLayout(1, 1, 1, "int8").bytes_per_token() == 2
    assert rm_compat.KVLayout(32, 8, 128, "bf16").bytes_per_token() == 131072


def test_product_carries_no_test_doubles():
    assert not hasattr(rm_compat, "LoopbackTransport")
    assert not hasattr(rm_compat, "check_kv_transport")
