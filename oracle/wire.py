"""Restatement of the reference's bf16 wire and /dev/shm handoff -- TEST INFRASTRUCTURE.

Follows connector/transport.py:29-43 (ser/deser), :80-101 (ShmTransport file
protocol), connector/rngd_kv.py:122-166 (save_kv_layer / wait_for_layer_load)
and serving/cluster.py:438-467 (_load_kv_now: f32 zero buffers, per-layer
load, unlink by prefix). It is both the byte-level oracle for the product's
frame codec and, timed, the CPU baseline of the handoff.
"""
import os
import pickle
import time

import numpy as np


def make_kv(seed, shape):
    """bf16-valued float32 N(0,1) arrays, the reference generator
    (bench/kv_tcp_bench.py:36-44: standard_normal, then bits >> 16 << 16)."""
    rng = np.random.default_rng(seed)
    x = rng.standard_normal(shape).astype(np.float32)
    return (x.view(np.uint32) >> 16 << 16).view(np.float32)


def ser(arr, wire="bf16"):
    """connector/transport.py:29-37."""
    a = np.ascontiguousarray(arr)
    if wire == "bf16":
        f = a if a.dtype == np.float32 else a.astype(np.float32)
        u = (f.view(np.uint32) >> 16).astype(np.uint16)
        return pickle.dumps({"bf16": u, "shape": a.shape}, protocol=4)
    return pickle.dumps(a.astype(np.float16), protocol=4)


def deser(buf):
    """connector/transport.py:39-43. Only ever called on blobs this process wrote."""
    o = pickle.loads(buf)
    if isinstance(o, dict) and "bf16" in o:
        return (o["bf16"].astype(np.uint32) << 16).view(np.float32).reshape(o["shape"])
    return o.astype(np.float32)


def shm_path(root, key):
    """connector/transport.py:89."""
    return os.path.join(root, key.replace("/", "__"))


def shm_push(root, key, buf):
    """connector/transport.py:90-94: write tmp.<pid>, flush, fsync, rename."""
    p = shm_path(root, key)
    tmp = p + f".tmp.{os.getpid()}"
    with open(tmp, "wb") as f:
        f.write(buf)
        f.flush()
        os.fsync(f.fileno())
    os.rename(tmp, p)


def shm_pull(root, key, timeout=5.0):
    """connector/transport.py:95-100: poll every 1 ms, then read."""
    p = shm_path(root, key)
    t0 = time.time()
    while not os.path.exists(p):
        if time.time() - t0 > timeout:
            raise TimeoutError(f"pull timeout: {key}")
        time.sleep(0.001)
    with open(p, "rb") as f:
        return f.read()


def save_request(root, req_id, k_frames, v_frames):
    """FullPrefillWorker._save_group -> save_kv_layer (serving/cluster.py:216-218,
    connector/rngd_kv.py:122-127): one k and one v blob per layer."""
    for i, (k, v) in enumerate(zip(k_frames, v_frames)):
        shm_push(root, f"{req_id}/layer.{i}/k", ser(k))
        shm_push(root, f"{req_id}/layer.{i}/v", ser(v))


def load_request(root, req_id, n_layers, n_kv, hd, S, timeout=5.0):
    """DecodeWorkerBase._load_kv_now (serving/cluster.py:438-467) with
    wait_for_layer_load (connector/rngd_kv.py:139-166): f32 zeros
    K [nl,NKV,HD,S] / V [nl,NKV,S,HD], pull + deser + place per layer, then
    unlink the request's files."""
    K = np.zeros((n_layers, n_kv, hd, S), np.float32)
    V = np.zeros((n_layers, n_kv, S, hd), np.float32)
    for i in range(n_layers):
        K[i][:] = deser(shm_pull(root, f"{req_id}/layer.{i}/k", timeout))
        V[i][:] = deser(shm_pull(root, f"{req_id}/layer.{i}/v", timeout))
    for f in os.listdir(root):
        if f.startswith(req_id + "__"):
            try:
                os.unlink(os.path.join(root, f))
            except OSError:
                pass
    return K, V


def frames_from_prefill(kv_tok, P, S):
    """Reference frames for one request from token-major prefill KV.

    kv_tok: float32 [L, 2, T, Hkv, D] (bf16-valued). Returns K frames
    [L, Hkv, D, S] and V frames [L, Hkv, S, D], zero for t >= P
    (engines/prefill_full.py:378-379)."""
    L, _, T, H, D = kv_tok.shape
    K = np.zeros((L, H, D, S), np.float32)
    V = np.zeros((L, H, S, D), np.float32)
    K[:, :, :, :P] = np.transpose(kv_tok[:, 0, :P], (0, 2, 3, 1))
    V[:, :, :P, :] = np.transpose(kv_tok[:, 1, :P], (0, 2, 1, 3))
    return K, V


def cpu_shm_handoff(root, req_id, K_frames, V_frames):
    """The whole reference CPU path for one request: save (ser + push), then
    load (pull + deser + place + unlink). Returns (K, V, seconds)."""
    L, H, D, S = K_frames.shape
    t0 = time.perf_counter()
    save_request(root, req_id, K_frames, V_frames)
    K, V = load_request(root, req_id, L, H, D, S)
    return K, V, time.perf_counter() - t0
