"""The handoff through pinned host memory: prefill KV -> host frame -> paged cache.

The reference moves every request through host memory: the prefill side pads
each layer group to S columns and downloads it (engines/prefill_full.py:366-384),
the wire carries the S-wide frame (connector/transport.py:29-37, 80-101), and the
decode side uploads and writes it into its cache (engines/decode_batch.py:305-377).
HostStagedHandoff does the same for a batch of requests on one GPU, layer by
layer, with nothing synchronising the host between requests:

  mode "kernel" (the default, and the faster one here):
    save stream   per layer, one launch for every request: pack_kernel stores
                  the layer's valid K and V columns (K in whole 64-token
                  tiles) straight into each request's pinned host frame
                  (pinned memory is device-visible, so the kernel's stores
                  are the device->host leg), then an event;
    host threads  meanwhile write the frame's zero tail (K columns >=
                  round64(P), V rows >= P) into the same pinned frame
                  (pdk_host_zero_frame_tail): host memory takes those bytes
                  at its own bandwidth instead of the link;
    load stream   per layer, one launch for every request: wait for that
                  layer's pack event, then scatter_kernel reads the layer's
                  valid columns from the pinned frames (its loads are the
                  host->device leg) and writes the paged cache blocks.
  mode "dma":
    the current stream packs into device frames; the DMA engines copy each
    layer to the pinned frame (save stream) and back into a second device
    frame (load stream); the current stream scatters from it. This is the
    reference's download / upload shape with copy engines.

In both modes the pinned frame of a request ends up holding exactly the wire
payload of every layer (K [Hkv, D, S] then V [Hkv, S, D], columns >= P zero),
and the cache holds what pdk_scatter_paged writes from that frame. The caller's
current stream waits for the last scatter, so work issued after run() sees the
cache; run() returns once the host's part is done.

Measured on MI355X (8 Llama-3.1-8B requests, P uniform in [64, 512]): the
host link carries about 55 GB/s in total whichever way the bytes go (copies
both ways at once share it). With the device writing whole S-wide frames
(537 MB down, 226 MB up) the batch took 14.9 ms; per-layer DMA copies of
whole frames both ways took 25-35 ms.
"""
import ctypes
import os
import threading

import numpy as np
import torch

from .. import _lib
from .._lib import PDK_COPY_D2H, PDK_COPY_H2D, PDK_PACK_NARROW, PDK_EVENT_SYNC, PackReq, ScatterReq
from ..hip import EventArray, PinnedBuffer
from .handoff import _as_layers, _check_cache, _need

MODES = ("kernel", "dma")


class HostStagedHandoff:
    """Pinned host frames for up to ``max_requests`` requests of one model shape."""

    def __init__(self, n_layers, n_kv_heads, head_dim, S, max_requests, device=None,
                 mode="kernel", host_threads=None):
        if mode not in MODES:
            raise ValueError(f"mode must be one of {MODES}, got {mode!r}")
        if mode == "kernel" and not 1 <= max_requests <= _lib.PDK_MAX_BATCH:
            raise ValueError(f"kernel mode batches up to {_lib.PDK_MAX_BATCH} requests per "
                             f"launch; got max_requests={max_requests}")
        self.L, self.H, self.D, self.S = n_layers, n_kv_heads, head_dim, S
        self.max_requests, self.mode = max_requests, mode
        self.device = torch.device(device or "cuda")
        self.F = n_kv_heads * head_dim * S                 # elements of one K (or V) frame
        self.layer_bytes = 2 * self.F * 2
        self.frame_bytes = n_layers * self.layer_bytes
        self.pinned = PinnedBuffer(max_requests * self.frame_bytes)
        if mode == "kernel":
            # One event per layer for the whole batch's pack, and one for the
            # end of the last run's scatters (a later run's host zeros may not
            # land where those scatters still read).
            self.ev_layer = EventArray(n_layers)
            self.ev_read = EventArray(1, PDK_EVENT_SYNC)
        else:
            self.ev_save = [EventArray(n_layers) for _ in range(max_requests)]
            self.ev_read = None
        self.slot_P = [None] * max_requests
        self.host_threads = int(host_threads or min(8, os.cpu_count() or 1))
        self.ev_load = [EventArray(n_layers) for _ in range(max_requests)] if mode == "dma" else None
        if mode == "dma":
            shape = (max_requests, n_layers, 2, self.F)
            self.out_frames = torch.empty(shape, dtype=torch.bfloat16, device=self.device)
            self.in_frames = torch.empty(shape, dtype=torch.bfloat16, device=self.device)
            self.ev_pack = [EventArray(n_layers) for _ in range(max_requests)]
        # Two side streams per process at most (the hardware has four queues
        # per process, and the caller's stream is a third).
        from ..connector.gpu_stage import side_stream
        self.save_stream = side_stream(self.device, "save")
        self.load_stream = side_stream(self.device, "load")

    def host_ptr(self, r):
        return self.pinned.ptr + r * self.frame_bytes

    def host_frame(self, r):
        """Request slot r's pinned frame as uint16 [L, 2, F] (the wire payloads)."""
        return self.pinned.view(np.uint16, r * self.frame_bytes,
                                self.frame_bytes // 2).reshape(self.L, 2, self.F)

    def _pack_req(self, k, v, P, dst, flags=0):
        _need(k, "k")
        _need(v, "v")
        k, v = _as_layers(k, v)
        if (k.shape[0], k.shape[2], k.shape[3]) != (self.L, self.H, self.D):
            raise ValueError(f"prefill KV {tuple(k.shape)} does not match "
                             f"(L={self.L}, Hkv={self.H}, D={self.D})")
        if not 0 <= P <= min(k.shape[1], self.S):
            raise ValueError(f"num_tokens={P} outside [0, min(T={k.shape[1]}, S={self.S})]")
        return PackReq(k.data_ptr(), v.data_ptr(), dst, k.stride(0), k.stride(1), int(P), flags)

    def _scatter_req(self, table, P, src):
        _need(table, "table", torch.int32)
        if not table.is_contiguous() or table.numel() < (P + 15) // 16:
            raise ValueError(f"block table must be contiguous with >= {(P + 15) // 16} entries "
                             f"for {P} tokens, got {table.numel()}")
        return ScatterReq(src, table.data_ptr(), int(P), table.numel())

    def run(self, requests, cache_k, cache_v):
        """requests: list of (k, v, num_tokens, table) -- k, v CUDA bf16 [L, T, Hkv, D]
        (token-major, [Hkv, D] contiguous), table a device int32 block table.
        Request i uses pinned slot i. Returns at once; the current stream waits."""
        if not 1 <= len(requests) <= self.max_requests:
            raise ValueError(f"1 to {self.max_requests} requests per run, got {len(requests)}")
        cache_k, cache_v = _check_cache(cache_k, cache_v)
        if cache_k.shape[0] != self.L:
            raise ValueError(f"cache has {cache_k.shape[0]} layers, frames {self.L}")
        nb = cache_k.shape[1]
        lib = _lib.lib()
        cur = torch.cuda.current_stream(self.device)
        L, S, H, D = self.L, self.S, self.H, self.D
        packs, scats = [], []
        kernel = self.mode == "kernel"
        for r, (k, v, P, table) in enumerate(requests):
            dst = self.host_ptr(r) if kernel else self.out_frames[r].data_ptr()
            packs.append(self._pack_req(k, v, P, dst, PDK_PACK_NARROW if kernel else 0))
            src = self.host_ptr(r) if self.mode == "kernel" else self.in_frames[r].data_ptr()
            scats.append(self._scatter_req(table, P, src))

        def ok(rc, what):
            if rc:
                raise _lib.PdkError(rc, what, _lib.last_error())

        n = len(requests)
        if kernel:
            # The zero tails, on host threads, while the device packs and
            # scatters. A slot's new zeros start at its new P: if an earlier,
            # longer request's scatter may still read that slot there, wait
            # for the last run's scatters first.
            lengths = [int(P) for _, _, P, _ in requests]
            wait = any(self.slot_P[r] is not None and lengths[r] < self.slot_P[r]
                       for r in range(n))
            errors = []

            def zero_tails():
                try:
                    if wait:
                        self.ev_read.sync(0)
                    for r, P in enumerate(lengths):
                        ok(lib.pdk_host_zero_frame_tail(ctypes.c_void_p(self.host_ptr(r)), L, H,
                                                        D, S, P, self.host_threads),
                           "pdk_host_zero_frame_tail")
                except BaseException as e:      # re-raised on the calling thread
                    errors.append(e)

            filler = threading.Thread(target=zero_tails, name="kv-zero-tails")
            filler.start()
            try:
                self.save_stream.wait_stream(cur)
                self.load_stream.wait_stream(cur)
                # Layer by layer, all requests in one launch each way: 2 L
                # launches for the batch.
                ok(lib.pdk_pack_kv_layerwise((PackReq * n)(*packs), n, L, S, H, D,
                                             self.ev_layer.ptr, self.save_stream.cuda_stream),
                   "pdk_pack_kv_layerwise")
                ok(lib.pdk_scatter_paged_layerwise((ScatterReq * n)(*scats), n, L, S, H, D,
                                                   cache_k.data_ptr(), cache_v.data_ptr(),
                                                   cache_k.stride(0), nb, self.ev_layer.ptr,
                                                   self.load_stream.cuda_stream),
                   "pdk_scatter_paged_layerwise")
                ok(lib.pdk_event_record(self.ev_read[0], self.load_stream.cuda_stream),
                   "pdk_event_record")
                cur.wait_stream(self.load_stream)
                cur.wait_stream(self.save_stream)
            finally:
                filler.join()
            if errors:
                raise errors[0]
            for r, P in enumerate(lengths):
                self.slot_P[r] = P
            return
        # dma: packs and scatters on the current stream (all packs first, so no
        # pack waits behind a scatter), copies on the two side streams.
        self.save_stream.wait_stream(cur)
        self.load_stream.wait_stream(cur)
        st = cur.cuda_stream
        for r, pr in enumerate(packs):
            ok(lib.pdk_pack_kv_layerwise(ctypes.byref(pr), 1, L, S, H, D, self.ev_pack[r].ptr, st),
               "pdk_pack_kv_layerwise")
        for r in range(len(requests)):
            ok(lib.pdk_copy_layers(ctypes.c_void_p(self.host_ptr(r)),
                                   ctypes.c_void_p(self.out_frames[r].data_ptr()),
                                   self.layer_bytes, L, PDK_COPY_D2H, self.ev_pack[r].ptr,
                                   self.ev_save[r].ptr, self.save_stream.cuda_stream),
               "pdk_copy_layers (D2H)")
        for r in range(len(requests)):
            ok(lib.pdk_copy_layers(ctypes.c_void_p(self.in_frames[r].data_ptr()),
                                   ctypes.c_void_p(self.host_ptr(r)), self.layer_bytes, L,
                                   PDK_COPY_H2D, self.ev_save[r].ptr, self.ev_load[r].ptr,
                                   self.load_stream.cuda_stream), "pdk_copy_layers (H2D)")
        for r, sr in enumerate(scats):
            ok(lib.pdk_scatter_paged_layerwise(ctypes.byref(sr), 1, L, S, H, D, cache_k.data_ptr(),
                                               cache_v.data_ptr(), cache_k.stride(0), nb,
                                               self.ev_load[r].ptr, st),
               "pdk_scatter_paged_layerwise")
        cur.wait_stream(self.save_stream)
        cur.wait_stream(self.load_stream)

    def link_bytes(self, lengths):
        """Bytes one run() moves over the host link. "kernel": the valid columns
        each way (K rows in whole 64-token tiles on the way down); "dma": whole
        S-wide frames each way."""
        if self.mode == "dma":
            return 2 * len(lengths) * self.frame_bytes
        half = self.L * self.H * self.D * 2              # one token of K (or V), all layers
        down = sum((min((P + 63) // 64 * 64, self.S) + P) * half for P in lengths)
        up = sum(2 * P * half for P in lengths)
        return down + up

    def close(self):
        torch.cuda.current_stream(self.device).synchronize()
        if self.ev_read is not None:
            self.ev_read.close()
            self.ev_layer.close()
        for arrs in (getattr(self, "ev_save", None), self.ev_load, getattr(self, "ev_pack", None)):
            for e in arrs or ():
                e.close()
        self.pinned.close()
