"""The connector's device path on the GPU, against the oracle's host path.

  save  CUDA bf16 token-major KV -> files byte-identical to the reference
        protocol's files for the same KV (oracle.wire: ser + shm_push);
  load  the reference protocol's files -> paged cache bit-identical to the
        oracle's scatter; device frames returned equal the payloads;
  both  device save then device load, through select_transport("shm").
"""
import os
import tempfile

import numpy as np
import pytest
import torch

from oracle import native as orc
from oracle import wire as owire
from tests._util import rand_bf16, to_dev, to_host

pytestmark = pytest.mark.gpu

L, H, D = 4, 8, 128


def _tmpdir():
    return tempfile.TemporaryDirectory(dir="/dev/shm" if os.access("/dev/shm", os.W_OK) else None)


def _frames_f32(k_bits, v_bits, P, S):
    """Reference frames [L, H, D, S] / [L, H, S, D] as float32 (what the reference ships)."""
    frame = orc.pack_kv(k_bits, v_bits, P, S)
    w = lambda u: (u.astype(np.uint32) << 16).view(np.float32)   # noqa: E731
    return (w(frame[:, 0]).reshape(L, H, D, S), w(frame[:, 1]).reshape(L, H, S, D), frame)


@pytest.mark.parametrize("T,P,S", [(512, 512, 512), (300, 237, 512), (64, 17, 64)])
def test_device_save_files_equal_reference(cuda, T, P, S):
    from rngd_pd_amd.connector import transport as kv
    from rngd_pd_amd.connector.rngd_kv import KVConnectorRole, RngdKVConnector
    rng = np.random.default_rng(T + P)
    k, v = rand_bf16(rng, (L, T, H, D)), rand_bf16(rng, (L, T, H, D))
    Kf, Vf, _ = _frames_f32(k, v, P, S)
    with _tmpdir() as a, _tmpdir() as b:
        conn = RngdKVConnector(KVConnectorRole.WORKER, req_id="g1", transport=kv.ShmTransport(a),
                               n_layers=L, frame_tokens=S)
        dk, dv = to_dev(k), to_dev(v)
        for i in range(L):
            conn.save_kv_layer(f"layer.{i}", (dk[i], dv[i]), num_tokens=P)
        conn.wait_for_save()
        assert conn.get_finished(set()) == ({"g1"}, None)
        conn.close()
        owire.save_request(b, "g1", Kf, Vf)
        names = sorted(os.listdir(b))
        assert sorted(os.listdir(a)) == names and len(names) == 2 * L
        for n in names:
            with open(os.path.join(a, n), "rb") as fa, open(os.path.join(b, n), "rb") as fb:
                assert fa.read() == fb.read(), n


@pytest.mark.parametrize("P,S", [(512, 512), (237, 512), (17, 64)])
def test_device_load_matches_oracle_scatter(cuda, P, S):
    from rngd_pd_amd.connector import transport as kv
    from rngd_pd_amd.connector.rngd_kv import KVConnectorRole, RngdKVConnector
    from rngd_pd_amd.engines.paged_cache import PagedKVCache
    rng = np.random.default_rng(P)
    k, v = rand_bf16(rng, (L, S, H, D)), rand_bf16(rng, (L, S, H, D))
    Kf, Vf, frame = _frames_f32(k, v, P, S)
    nb = 2 * ((S + 15) // 16)
    cache = PagedKVCache(L, nb, H, D, device=cuda, seed=P)
    with _tmpdir() as root:
        owire.save_request(root, "g2", Kf, Vf)          # the reference's files
        conn = RngdKVConnector(KVConnectorRole.WORKER, req_id="g2", transport=kv.ShmTransport(root),
                               n_layers=L)
        conn.register_kv_caches(cache.view("g2", P, S))
        conn.bind_connector_metadata(conn.build_connector_meta(None))
        conn.start_load_kv()
        views = [conn.wait_for_layer_load(f"layer.{i}") for i in range(L)]
        torch.cuda.synchronize()
        for i, (fk, fv) in enumerate(views):
            np.testing.assert_array_equal(to_host(fk).reshape(-1), frame[i, 0])
            np.testing.assert_array_equal(to_host(fv).reshape(-1), frame[i, 1])
        want_k = np.zeros((L, nb, H, 16, D), np.uint16)
        want_v = np.zeros((L, nb, H, D, 16), np.uint16)
        orc.scatter_paged(frame, np.asarray(cache.blocks("g2"), np.int32), P, S, H, D, want_k, want_v)
        np.testing.assert_array_equal(to_host(cache.k), want_k)
        np.testing.assert_array_equal(to_host(cache.v), want_v)
        conn.close()


@pytest.mark.parametrize("nl,P", [(4, 333), (32, 512)])
def test_device_to_device_through_selected_shm(cuda, monkeypatch, nl, P):
    """Device save -> /dev/shm -> device load through select_transport("shm"); at
    nl=32, P=S=512 this is one whole Llama-3.1-8B request (64 MiB on the wire).
    The load consumes the request's files and nothing else: files of another
    request (one whose id extends this one's) survive the load and close()."""
    from rngd_pd_amd.connector import transport as kv
    from rngd_pd_amd.connector.rngd_kv import KVConnectorRole, RngdKVConnector
    from rngd_pd_amd.engines.paged_cache import PagedKVCache
    S = 512
    rng = np.random.default_rng(77 + nl)
    k, v = rand_bf16(rng, (nl, S, H, D)), rand_bf16(rng, (nl, S, H, D))
    with _tmpdir() as root:
        monkeypatch.setenv("PD_SHM_ROOT", root)
        monkeypatch.setenv("AIRM_KV_TRANSPORT", "shm")
        kv.reset_selection()
        pf = RngdKVConnector(KVConnectorRole.WORKER, req_id="g3", n_layers=nl, frame_tokens=S)
        dk, dv = to_dev(k), to_dev(v)
        for i in range(nl):
            pf.save_kv_layer(f"layer.{i}", torch.stack([dk[i], dv[i]]), num_tokens=P)
        pf.wait_for_save()
        pf.close()
        decoys = ["g33__layer.0__k", "other__layer.0__v"]
        for name in decoys:
            with open(os.path.join(root, name), "wb") as f:
                f.write(b"not mine")
        assert len(os.listdir(root)) == 2 * nl + len(decoys)
        cache = PagedKVCache(nl, 2 * ((S + 15) // 16), H, D, device=cuda, seed=1)
        dc = RngdKVConnector(KVConnectorRole.WORKER, req_id="g3", n_layers=nl)
        dc.register_kv_caches(cache.view("g3", P, S))
        dc.start_load_kv()
        for i in range(nl):
            dc.wait_for_layer_load(f"layer.{i}")
        back = cache.read_frame("g3", P, S)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(to_host(back), orc.pack_kv(k, v, P, S))
        assert sorted(os.listdir(root)) == sorted(decoys)     # consumed, decoys kept
        dc.close()
        assert sorted(os.listdir(root)) == sorted(decoys)
        kv.reset_selection()


def test_device_to_device_through_tcp_relay(cuda, monkeypatch):
    """The device path over the native tcp relay: save packs into pinned
    memory and pushes header + payload + trailer in one send (CRC-32 on);
    load receives each blob straight into pinned memory and scatters it. The
    relay's blobs are the reference protocol's files byte for byte, and the
    paged cache holds the oracle's frame."""
    from rngd_pd_amd.connector import transport as kv
    from rngd_pd_amd.connector.rngd_kv import KVConnectorRole, RngdKVConnector
    from rngd_pd_amd.connector.tcp import TcpKVServer, TcpTransport
    from rngd_pd_amd.engines.paged_cache import PagedKVCache
    S, P = 512, 301
    rng = np.random.default_rng(78)
    k, v = rand_bf16(rng, (L, S, H, D)), rand_bf16(rng, (L, S, H, D))
    srv = TcpKVServer(0, "127.0.0.1").start()
    port = srv.wait_ready()
    try:
        t_pre = TcpTransport(remote=("127.0.0.1", port))
        pf = RngdKVConnector(KVConnectorRole.WORKER, req_id="g4", transport=t_pre, n_layers=L,
                             frame_tokens=S)
        dk, dv = to_dev(k), to_dev(v)
        for i in range(L):
            pf.save_kv_layer(f"layer.{i}", (dk[i], dv[i]), num_tokens=P)
        pf.wait_for_save()
        pf.close()
        st = srv.stats
        assert st["pushed"] == 2 * L and st["crc_errors"] == 0
        # One layer's blobs against the reference protocol's files for the same KV.
        Kf, Vf, frame = _frames_f32(k, v, P, S)
        with _tmpdir() as ref:
            owire.save_request(ref, "g4", Kf, Vf)
            for name in ("layer.0/k", "layer.0/v"):
                blob = bytes(t_pre.pull(f"g4/{name}", timeout=5))
                with open(os.path.join(ref, "g4__" + name.replace("/", "__")), "rb") as f:
                    assert blob == f.read(), name
                t_pre.push(f"g4/{name}", blob)                   # put it back for the load
        t_dec = TcpTransport(remote=("127.0.0.1", port))
        cache = PagedKVCache(L, 64, H, D, device=cuda, seed=2)
        dc = RngdKVConnector(KVConnectorRole.WORKER, req_id="g4", transport=t_dec, n_layers=L)
        dc.register_kv_caches(cache.view("g4", P, S))
        dc.start_load_kv()
        for i in range(L):
            dc.wait_for_layer_load(f"layer.{i}")
        back = cache.read_frame("g4", P, S)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(to_host(back), frame)
        dc.close()
        assert srv.stats["keys"] == 0
        t_pre.close()
        t_dec.close()
    finally:
        srv.stop()
