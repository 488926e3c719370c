"""Same-GPU handoff through hipIpc handles: prefill and decode as two processes
on one device, with the frame never leaving HBM.

This is the "same-GPU hipIpc handles for the decode process" leg of the handoff.
It stands in for the host round trip of the shm path (files written at
connector/transport.py:80-101, read and placed at connector/rngd_kv.py:139-166)
when producer and consumer share the GPU. The connector surface is unchanged:
select it with AIRM_KV_TRANSPORT=ipc (or pass an IpcTransport), then call
save_kv_layer / wait_for_save on the prefill side and register_kv_caches(view)
/ start_load_kv / wait_for_layer_load on the decode side.

Producer. An IpcFramePool owns one device allocation of n_slots request frames
[L][2][Hkv*D*S] bf16 (the layout of the shm wire payload), kept below 2 GiB
because IPC mappings on this platform must be. An IpcSaver (one request) packs
each saved layer into its slot on the process's save stream, writing only the
valid columns (the consumer's scatter never reads the S-wide zero tail). wait() waits on
the host for those packs to finish, then publishes the descriptor "<req>/ipc"
(a small JSON file) with the shm publish sequence (tmp + fsync + rename): a
descriptor only ever names a complete frame. (Interprocess events, which would
let the consumer's stream wait instead, are refused by this platform's IPC
mode: hipIpcGetEventHandle returns invalid argument.) The slot returns to the
pool once the consumer has published "<req>/ipc.done".

Consumer. An IpcLoader (one request) pulls the descriptor with the shm pull
(1 ms polling, PD_KV_PULL_TIMEOUT) and opens the pool's handle, which stays
cached for the process. One scatter launch moves every layer from the
producer's frame into the paged cache. The host waits for that scatter, then
publishes ".done". The consumer deletes the descriptor; the producer deletes
".done" when it reclaims the slot.
"""
import json
import os
import threading
import time
from collections import deque

import torch

from .. import _lib
from .._lib import PDK_EVENT_SYNC
from ..hip import DeviceBuffer, Event
from ..kernels import handoff as _h
from .gpu_stage import side_stream
from .transport import ShmTransport

IPC_LIMIT = 2 << 30          # bytes per exported allocation on this platform


def frame_nbytes(n_layers, n_kv_heads, head_dim, S):
    return n_layers * 2 * n_kv_heads * head_dim * S * 2


class IpcFramePool:
    """Producer-side device frame slots exported through one IPC handle."""

    def __init__(self, transport, n_layers, n_kv_heads, head_dim, S, n_slots=None, device=None):
        self.t = transport
        self.L, self.H, self.D, self.S = n_layers, n_kv_heads, head_dim, S
        self.device = torch.device(device or "cuda")
        self.frame_bytes = frame_nbytes(n_layers, n_kv_heads, head_dim, S)
        if n_slots is None:
            n_slots = int(os.environ.get("PD_IPC_SLOTS", "8"))
        n_slots = max(1, min(n_slots, (IPC_LIMIT - 1) // self.frame_bytes))
        if n_slots * self.frame_bytes >= IPC_LIMIT:
            raise ValueError(f"one {self.frame_bytes}-byte frame does not fit a {IPC_LIMIT}-byte "
                             f"IPC allocation")
        self.n_slots = n_slots
        with torch.cuda.device(self.device):
            self.buf = DeviceBuffer(n_slots * self.frame_bytes)
            self.events = [Event(PDK_EVENT_SYNC) for _ in range(n_slots)]
        self.mem_handle = self.buf.ipc_handle().hex()
        self._free = deque(range(n_slots))
        self._out = {}                               # req_id -> slot awaiting the consumer
        self._lock = threading.Lock()

    def frame_ptr(self, slot):
        return self.buf.ptr + slot * self.frame_bytes

    def _reclaim(self):
        for req, slot in list(self._out.items()):
            done = self.t._path(f"{req}/ipc.done")
            if os.path.exists(done):
                os.unlink(done)
                del self._out[req]
                self._free.append(slot)

    def acquire(self, req_id, timeout=None):
        """A free slot for ``req_id``; waits (1 ms polling) for a consumer to release one."""
        if timeout is None:
            timeout = float(os.environ.get("PD_KV_PULL_TIMEOUT", "5"))
        t0 = time.time()
        while True:
            with self._lock:
                self._reclaim()
                if self._free:
                    slot = self._free.popleft()
                    self._out[req_id] = slot
                    return slot
            if time.time() - t0 > timeout:
                raise TimeoutError(f"ipc frame pool full: no consumer released a slot within "
                                   f"{timeout} s")
            time.sleep(0.001)

    def outstanding(self):
        with self._lock:
            self._reclaim()
            return dict(self._out)

    def close(self, timeout=5.0):
        """Wait (bounded) for consumers to release their slots, then free the pool."""
        t0 = time.time()
        while self.outstanding() and time.time() - t0 < timeout:
            time.sleep(0.001)
        torch.cuda.synchronize(self.device)
        for e in self.events:
            e.close()
        self.buf.close()


class IpcSaver:
    """One request's layers packed into a pool slot; wait() publishes the descriptor."""

    def __init__(self, transport, req_id, pool):
        self.t, self.req_id, self.pool = transport, req_id, pool
        self.slot = pool.acquire(req_id)
        self.stream = side_stream(pool.device)
        self.P = None
        self._layers = set()
        self._published = False

    def save(self, layer_name, k, v, num_tokens):
        """k, v CUDA bf16 [T, Hkv, D] (token-major), T >= num_tokens."""
        li = int(layer_name.split(".")[-1])
        pool = self.pool
        if not 0 <= li < pool.L:
            raise ValueError(f"{layer_name}: layer index outside [0, {pool.L})")
        if self.P is not None and num_tokens != self.P:
            raise ValueError(f"num_tokens {num_tokens} differs from the request's {self.P}")
        if self._published:
            raise RuntimeError(f"{self.req_id}: save after wait_for_save")
        self.P = int(num_tokens)
        producer = torch.cuda.current_stream(pool.device)
        self.stream.wait_stream(producer)
        with torch.cuda.stream(self.stream):
            for t in (k, v):
                t.record_stream(self.stream)
            layer_bytes = pool.frame_bytes // pool.L
            # Narrow: the consumer's scatter reads only columns < P, so the
            # S-wide zero tail would be bytes written that nobody reads.
            _h.pack_kv(k, v, self.P, pool.S, stream=self.stream,
                       frame_ptr=pool.frame_ptr(self.slot) + li * layer_bytes, narrow=True)
        self._layers.add(li)

    def wait(self):
        if self._published:
            return
        pool = self.pool
        if len(self._layers) != pool.L:
            missing = sorted(set(range(pool.L)) - self._layers)
            raise RuntimeError(f"{self.req_id}: layers {missing[:4]}... were not saved")
        ev = pool.events[self.slot]
        ev.record(self.stream.cuda_stream)
        ev.sync()                                    # the frame is complete in HBM
        desc = {"v": 1, "pool": pool.mem_handle, "pool_bytes": pool.buf.nbytes,
                "offset": self.slot * pool.frame_bytes, "L": pool.L, "H": pool.H,
                "D": pool.D, "S": pool.S, "P": self.P, "pid": os.getpid(),
                "columns": "valid"}         # columns >= P of the frame are not written
        self.t.push(f"{self.req_id}/ipc", json.dumps(desc).encode())
        self._published = True

    def saved_layers(self):
        return {f"layer.{i}" for i in self._layers}

    def close(self):
        self.wait()


# Consumer-side mappings stay open for the process: a producer reuses its
# slots, so one mapping per pool serves every later request.
_OPEN_MEM = {}
_OPEN_LOCK = threading.Lock()


def _open_pool(handle_hex, nbytes):
    with _OPEN_LOCK:
        buf = _OPEN_MEM.get(handle_hex)
        if buf is None:
            buf = _OPEN_MEM[handle_hex] = DeviceBuffer.from_ipc(bytes.fromhex(handle_hex), nbytes)
        return buf


def close_opened():
    """Unmap every producer pool this process opened."""
    with _OPEN_LOCK:
        for buf in _OPEN_MEM.values():
            buf.close()
        _OPEN_MEM.clear()


class IpcLoader:
    """Consumer side of one request: the producer's frame -> the paged cache, in HBM."""

    def __init__(self, transport, req_id, view, n_layers, n_kv_heads, head_dim, device=None,
                 timeout=5.0):
        self.t, self.req_id, self.view = transport, req_id, view
        self.L, self.H, self.D = n_layers, n_kv_heads, head_dim
        self.device = torch.device(device or "cuda")
        self.timeout = timeout
        self.stream = side_stream(self.device, "load")
        self._loaded = False

    def _load_all(self):
        desc = json.loads(self.t.pull(f"{self.req_id}/ipc", timeout=self.timeout))
        os.unlink(self.t._path(f"{self.req_id}/ipc"))
        if (desc["L"], desc["H"], desc["D"]) != (self.L, self.H, self.D):
            raise ValueError(f"{self.req_id}: producer frame (L, Hkv, D) = "
                             f"{(desc['L'], desc['H'], desc['D'])}, cache "
                             f"{(self.L, self.H, self.D)}")
        S, P = desc["S"], desc["P"]
        view, cache = self.view, self.view.cache
        if P != view.num_tokens:
            raise ValueError(f"{self.req_id}: producer sent {P} tokens, the view holds "
                             f"{view.num_tokens}")
        pool = _open_pool(desc["pool"], desc["pool_bytes"])
        consumer = torch.cuda.current_stream(self.device)
        self.stream.wait_stream(consumer)
        st = self.stream.cuda_stream
        _lib.call("pdk_scatter_paged", pool.ptr + desc["offset"], view.table.data_ptr(),
                  view.table.numel(), self.L, P, S, self.H, self.D, cache.k.data_ptr(),
                  cache.v.data_ptr(), cache.k.stride(0), cache.num_blocks, st)
        done = Event(PDK_EVENT_SYNC)
        try:
            done.record(st)
            done.sync()                      # the producer's slot is read to the end
        finally:
            done.close()
        self.t.push(f"{self.req_id}/ipc.done", b"1")
        consumer.wait_stream(self.stream)
        self._loaded = True

    def load(self, layer_name, li):
        """Place the whole request on the first call; later layers are already there."""
        if not self._loaded:
            self._load_all()
        return None

    def close(self):
        pass


class IpcTransport(ShmTransport):
    """The shm file contract for small control files, frames through IPC on one GPU.

    Byte blobs (host arrays) still travel as shm files, so the transport serves
    every connector call; device KV goes through the frame pool."""

    name = "ipc"
    device_ipc = True

    def __init__(self, root=None, n_slots=None):
        from ..paths import SHM_ROOT
        super().__init__(root or os.environ.get("PD_SHM_ROOT") or SHM_ROOT)
        self.n_slots = n_slots
        self._pools = {}
        self._lock = threading.Lock()

    def pool(self, n_layers, n_kv_heads, head_dim, S, device):
        key = (n_layers, n_kv_heads, head_dim, S, str(device))
        with self._lock:
            p = self._pools.get(key)
            if p is None:
                p = self._pools[key] = IpcFramePool(self, n_layers, n_kv_heads, head_dim, S,
                                                    self.n_slots, device)
            return p

    def close(self):
        with self._lock:
            pools, self._pools = list(self._pools.values()), {}
        for p in pools:
            p.close()


__all__ = ["IpcTransport", "IpcFramePool", "IpcSaver", "IpcLoader", "close_opened",
           "frame_nbytes"]
