"""Device-side save and load of the /dev/shm handoff.

FrameSaver (prefill side) replaces the download + encode + write of
engines/prefill_full.py:378-384 and serving/cluster.py:187-218:
  side stream: wait for the producer's stream -> pack one layer's valid
  columns straight into a pinned host slot (device-visible memory: the pack
  kernel's stores carry the download, with no device staging slot and no
  copy) -> event;
  one writer thread, in save order (the reference's single ordered writer):
  wait for the event -> write the frame's zero tail (columns >= P) into the
  slot on the host, so only valid columns cross the host link -> publish
  "<req>/<layer>/k" and ".../v" as header + payload + trailer straight from
  pinned memory (byte-identical to ser() of the same bf16 KV) -> free the slot.
  wait() is the wait_for_save fence: every file of the request is published.

FrameLoader (decode side) replaces wait_for_layer_load's pull + deser + place
(connector/rngd_kv.py:139-166) and the stage/stack/upload of
engines/decode_batch.py:305-351:
  pull the k and v files into a pinned slot, the payload landing 256-byte
  aligned -> check the envelope -> copy to the request's device frame (side
  stream) -> scatter the layer into the paged cache -> event that the caller's
  stream waits on, so attention issued after the load sees the cache.
Pinned memory is allocated (hipHostMalloc), never registered.
"""
import queue
import threading

import numpy as np
import torch

from .. import _lib
from ..hip import EventArray, PinnedBuffer
from ..kernels import handoff as _h
from . import wire as _wire

ALIGN = 256


def _align(x, a=ALIGN):
    return (x + a - 1) // a * a


_SIDE_STREAMS = {}
_SIDE_LOCK = threading.Lock()


def side_stream(device, role="save"):
    """The process-wide side stream of ``device`` for ``role`` ("save" or
    "load"). Every request's copies and kernels of that role share it: with one
    stream per request, requests would outnumber the hardware queues (4 per
    process here), and a queue shared with the compute stream would hold copies
    behind later compute kernels."""
    key = (torch.device(device).index or 0, role)
    with _SIDE_LOCK:
        st = _SIDE_STREAMS.get(key)
        if st is None:
            st = _SIDE_STREAMS[key] = torch.cuda.Stream(device=device)
        return st


class FrameSaver:
    """Asynchronous, ordered device -> /dev/shm saver for one request."""

    def __init__(self, transport, req_id, n_kv_heads, head_dim, S, device=None, n_slots=4):
        self.t, self.req_id = transport, req_id
        self.H, self.D, self.S = n_kv_heads, head_dim, S
        self.device = torch.device(device or "cuda")
        self.F = n_kv_heads * head_dim * S                # elements per K (or V) frame
        self.slot_bytes = 2 * self.F * 2
        self.n_slots = n_slots
        self.stream = side_stream(self.device)
        self.pinned = PinnedBuffer(n_slots * self.slot_bytes)
        self.events = EventArray(n_slots)
        self._free = queue.Queue()
        for i in range(n_slots):
            self._free.put(i)
        self._jobs = queue.Queue()
        self._error = None
        self._done = set()
        self._writer = threading.Thread(target=self._write_loop, name=f"kv-save-{req_id}",
                                        daemon=True)
        self._writer.start()
        # The envelope is computed once per shape, off the hot path.
        _wire.envelope((n_kv_heads, head_dim, S))
        _wire.envelope((n_kv_heads, S, head_dim))

    def save(self, layer_name, k, v, num_tokens):
        """Queue one layer: k, v CUDA bf16 [T, Hkv, D] (token-major), T >= num_tokens."""
        if self._error:
            raise self._error
        slot = self._free.get()
        producer = torch.cuda.current_stream(self.device)
        self.stream.wait_stream(producer)
        with torch.cuda.stream(self.stream):
            for t in (k, v):
                t.record_stream(self.stream)
            # The runtime's own device-to-host copy is a blit kernel under some
            # HIP builds; its 256 workgroups then wait for CUs whenever a prefill
            # GEMM fills the chip. Packing into the pinned slot needs one launch
            # of half as many workgroups and no device slot.
            _h.pack_kv(k, v, num_tokens, self.S, stream=self.stream,
                       frame_ptr=self.pinned.ptr + slot * self.slot_bytes, narrow=True)
            _lib.call("pdk_event_record", self.events[slot], self.stream.cuda_stream)
        self._jobs.put((slot, layer_name, int(num_tokens)))

    def _write_loop(self):
        while True:
            job = self._jobs.get()
            if job is None:
                self._jobs.task_done()
                return
            slot, layer, P = job
            try:
                if self._error is None:
                    self.events.sync(slot)
                    base = slot * self.slot_bytes
                    _lib.call("pdk_host_zero_frame_tail", self.pinned.ptr + base, 1, self.H,
                              self.D, self.S, P, 64, 1)
                    half = self.F * 2
                    kmv = self.pinned.memoryview(base, half)
                    vmv = self.pinned.memoryview(base + half, half)
                    self._push(f"{self.req_id}/{layer}/k", kmv, (self.H, self.D, self.S))
                    self._push(f"{self.req_id}/{layer}/v", vmv, (self.H, self.S, self.D))
                    self._done.add(layer)
            except BaseException as e:  # surfaced by save()/wait()
                self._error = e
            finally:
                self._free.put(slot)
                self._jobs.task_done()

    def _push(self, key, payload, shape):
        parts = _wire.encode_parts(payload, shape)
        if hasattr(self.t, "push_parts"):
            self.t.push_parts(key, parts)
        else:
            self.t.push(key, b"".join(bytes(p) for p in parts))

    def wait(self):
        """Block until every queued layer is published; re-raise a writer failure."""
        self._jobs.join()
        if self._error:
            raise self._error

    def saved_layers(self):
        return set(self._done)

    def close(self):
        try:
            self.wait()
        finally:
            self._jobs.put(None)
            self._writer.join(timeout=5)
            self.events.close()
            self.pinned.close()


class FrameLoader:
    """/dev/shm -> pinned -> device frame -> paged cache, layer by layer."""

    def __init__(self, transport, req_id, view, n_layers, n_kv_heads, head_dim, device=None,
                 n_slots=2, timeout=5.0):
        self.t, self.req_id, self.view = transport, req_id, view
        self.L, self.H, self.D, self.S = n_layers, n_kv_heads, head_dim, view.S
        self.P = view.num_tokens
        self.timeout = timeout
        self.device = torch.device(device or "cuda")
        self.F = self.H * self.D * self.S
        self.payload = self.F * 2
        kh, kt = _wire.envelope((self.H, self.D, self.S))
        vh, vt = _wire.envelope((self.H, self.S, self.D))
        self.env = {"k": (len(kh), len(kt)), "v": (len(vh), len(vt))}
        # Per blob: room for pad + header + payload + trailer, payload 256-byte aligned.
        self.blob_room = _align(max(len(kh), len(vh)) + self.payload + max(len(kt), len(vt)) + ALIGN)
        self.slot_bytes = 2 * self.blob_room
        self.n_slots = n_slots
        self.pinned = PinnedBuffer(n_slots * self.slot_bytes)
        self.events = EventArray(n_slots)
        self._used = [False] * n_slots
        self._next = 0
        self.frame = torch.empty((n_layers, 2, self.F), dtype=torch.bfloat16, device=self.device)
        self.stream = side_stream(self.device, "load")

    def _read_blob(self, key, which, base, shape):
        """Pull one blob into pinned memory at ``base``; returns the payload's pinned offset."""
        hlen, _ = self.env[which]
        pad = _align(hlen) - hlen
        # A transport that can receive into a buffer (shm reads the file, tcp
        # the socket) writes the blob straight into pinned memory. shm knows
        # the size first; tcp finds out on arrival and keeps a blob that does
        # not fit for the pull() below.
        size = self.t.pull_size(key, self.timeout) if hasattr(self.t, "pull_size") else None
        fits = size is None or pad + size <= self.blob_room
        n = None
        if hasattr(self.t, "pull_into") and fits:
            try:
                n = self.t.pull_into(key, self.pinned.memoryview(base + pad, self.blob_room - pad),
                                     timeout=self.timeout)
            except ValueError:
                n = None
        if n is not None:
            blob = self.pinned.memoryview(base + pad, n)
            rng = _wire.payload_range(blob, shape)
            if rng is not None:
                return base + pad + rng[0]
            data = _wire.decode_payload(bytes(blob), shape)
        else:
            data = _wire.decode_payload(self.t.pull(key, timeout=self.timeout), shape)
        dst = self.pinned.view(np.uint16, base + _align(hlen), data.size)
        dst[:] = data.reshape(-1)
        return base + _align(hlen)

    def load(self, layer_name, li):
        """Load one layer into the paged cache; returns its device frame views (k, v)."""
        slot = self._next
        self._next = (slot + 1) % self.n_slots
        if self._used[slot]:
            self.events.sync(slot)               # the slot's previous H2D has finished
        base = slot * self.slot_bytes
        koff = self._read_blob(f"{self.req_id}/{layer_name}/k", "k", base, (self.H, self.D, self.S))
        voff = self._read_blob(f"{self.req_id}/{layer_name}/v", "v", base + self.blob_room,
                               (self.H, self.S, self.D))
        consumer = torch.cuda.current_stream(self.device)
        self.stream.wait_stream(consumer)
        st = self.stream.cuda_stream
        fk, fv = self.frame[li, 0], self.frame[li, 1]
        _lib.call("pdk_memcpy_h2d", fk.data_ptr(), self.pinned.ptr + koff, self.payload, st)
        _lib.call("pdk_memcpy_h2d", fv.data_ptr(), self.pinned.ptr + voff, self.payload, st)
        cache = self.view.cache
        _lib.call("pdk_scatter_paged", self.frame[li].data_ptr(), self.view.table.data_ptr(),
                  self.view.table.numel(), 1, self.P, self.S, self.H, self.D,
                  cache.k[li].data_ptr(), cache.v[li].data_ptr(), cache.k.stride(0),
                  cache.num_blocks, st)
        _lib.call("pdk_event_record", self.events[slot], st)
        self._used[slot] = True
        consumer.wait_stream(self.stream)
        return (fk.view(self.H, self.D, self.S), fv.view(self.H, self.S, self.D))

    def close(self):
        torch.cuda.current_stream(self.device).synchronize()
        self.events.sync()
        self.events.close()
        self.pinned.close()


def is_device_tensor(x):
    return isinstance(x, torch.Tensor) and x.is_cuda


def split_device_kv(kv_layer):
    """(k, v) CUDA tensors from a (k, v) pair or a stacked [2, ...] tensor."""
    if isinstance(kv_layer, (tuple, list)) and len(kv_layer) == 2:
        return kv_layer[0], kv_layer[1]
    if kv_layer.shape[0] != 2:
        raise ValueError(f"expected stacked [2, ...] kv_layer, got {tuple(kv_layer.shape)}")
    return kv_layer[0], kv_layer[1]


def frame_bytes(n_kv_heads, head_dim, S):
    return 2 * n_kv_heads * head_dim * S * 2


__all__ = ["FrameSaver", "FrameLoader", "is_device_tensor", "split_device_kv", "frame_bytes"]
