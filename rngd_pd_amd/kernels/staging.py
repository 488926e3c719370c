"""The handoff through pinned host memory: prefill KV -> host frame -> paged cache.

The reference moves every request through host memory: the prefill side pads
each layer group to S columns and downloads it (engines/prefill_full.py:366-384),
the wire carries the S-wide frame (connector/transport.py:29-37, 80-101), and the
decode side uploads and writes it into its cache (engines/decode_batch.py:305-377).
HostStagedHandoff does the same for a batch of requests on one GPU, layer by
layer, with nothing synchronising the host between requests:

  mode "kernel" (the default, and the faster one here):
    save stream   per (request, layer): pack_kernel stores the layer's S-wide
                  K and V frames straight into the request's pinned host frame
                  (pinned memory is device-visible, so the kernel's stores are
                  the device->host leg), then an event;
    load stream   per (request, layer): wait for that event, then
                  scatter_kernel reads the layer's valid columns from the pinned
                  frame (its loads are the host->device leg) and writes the
                  paged cache blocks.
  mode "dma":
    the current stream packs into device frames; the DMA engines copy each
    layer to the pinned frame (save stream) and back into a second device
    frame (load stream); the current stream scatters from it. This is the
    reference's download / upload shape with copy engines.

In both modes the pinned frame of a request ends up holding exactly the wire
payload of every layer (K [Hkv, D, S] then V [Hkv, S, D], columns >= P zero),
and the cache holds what pdk_scatter_paged writes from that frame. The caller's
current stream waits for the last scatter, so work issued after run() sees the
cache. Measured on MI355X (8 Llama-3.1-8B requests, P uniform in [64, 512]):
the host link carries about 55 GB/s in total whichever way the bytes go
(copies both ways at once share it), so "kernel" mode, which crosses it with
S-wide frames one way and only the valid columns the other, takes 14.9 ms per
batch; per-layer DMA copies both ways took 35 ms.
"""
import ctypes

import numpy as np
import torch

from .. import _lib
from .._lib import PDK_COPY_D2H, PDK_COPY_H2D, PackReq, ScatterReq
from ..hip import EventArray, PinnedBuffer
from .handoff import _as_layers, _check_cache, _need

MODES = ("kernel", "dma")


class HostStagedHandoff:
    """Pinned host frames for up to ``max_requests`` requests of one model shape."""

    def __init__(self, n_layers, n_kv_heads, head_dim, S, max_requests, device=None,
                 mode="kernel"):
        if mode not in MODES:
            raise ValueError(f"mode must be one of {MODES}, got {mode!r}")
        self.L, self.H, self.D, self.S = n_layers, n_kv_heads, head_dim, S
        self.max_requests, self.mode = max_requests, mode
        self.device = torch.device(device or "cuda")
        self.F = n_kv_heads * head_dim * S                 # elements of one K (or V) frame
        self.layer_bytes = 2 * self.F * 2
        self.frame_bytes = n_layers * self.layer_bytes
        self.pinned = PinnedBuffer(max_requests * self.frame_bytes)
        self.ev_save = [EventArray(n_layers) for _ in range(max_requests)]
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

    def _pack_req(self, k, v, P, dst):
        _need(k, "k")
        _need(v, "v")
        k, v = _as_layers(k, v)
        if (k.shape[0], k.shape[2], k.shape[3]) != (self.L, self.H, self.D):
            raise ValueError(f"prefill KV {tuple(k.shape)} does not match "
                             f"(L={self.L}, Hkv={self.H}, D={self.D})")
        if not 0 <= P <= min(k.shape[1], self.S):
            raise ValueError(f"num_tokens={P} outside [0, min(T={k.shape[1]}, S={self.S})]")
        return PackReq(k.data_ptr(), v.data_ptr(), dst, k.stride(0), k.stride(1), int(P), 0)

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
        for r, (k, v, P, table) in enumerate(requests):
            dst = self.host_ptr(r) if self.mode == "kernel" else self.out_frames[r].data_ptr()
            packs.append(self._pack_req(k, v, P, dst))
            src = self.host_ptr(r) if self.mode == "kernel" else self.in_frames[r].data_ptr()
            scats.append(self._scatter_req(table, P, src))

        def ok(rc, what):
            if rc:
                raise _lib.PdkError(rc, what, _lib.last_error())

        if self.mode == "kernel":
            self.save_stream.wait_stream(cur)
            self.load_stream.wait_stream(cur)
            st_save, st_load = self.save_stream.cuda_stream, self.load_stream.cuda_stream
            for r, pr in enumerate(packs):
                ok(lib.pdk_pack_kv_layerwise(ctypes.byref(pr), L, S, H, D, self.ev_save[r].ptr,
                                             st_save), "pdk_pack_kv_layerwise")
            for r, sr in enumerate(scats):
                ok(lib.pdk_scatter_paged_layerwise(ctypes.byref(sr), L, S, H, D,
                                                   cache_k.data_ptr(), cache_v.data_ptr(),
                                                   cache_k.stride(0), nb, self.ev_save[r].ptr,
                                                   st_load), "pdk_scatter_paged_layerwise")
            cur.wait_stream(self.load_stream)
            cur.wait_stream(self.save_stream)
            return
        # dma: packs and scatters on the current stream (all packs first, so no
        # pack waits behind a scatter), copies on the two side streams.
        self.save_stream.wait_stream(cur)
        self.load_stream.wait_stream(cur)
        st = cur.cuda_stream
        for r, pr in enumerate(packs):
            ok(lib.pdk_pack_kv_layerwise(ctypes.byref(pr), L, S, H, D, self.ev_pack[r].ptr, st),
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
            ok(lib.pdk_scatter_paged_layerwise(ctypes.byref(sr), L, S, H, D, cache_k.data_ptr(),
                                               cache_v.data_ptr(), cache_k.stride(0), nb,
                                               self.ev_load[r].ptr, st),
               "pdk_scatter_paged_layerwise")
        cur.wait_stream(self.save_stream)
        cur.wait_stream(self.load_stream)

    def link_bytes(self, lengths):
        """Bytes one run() moves over the host link: S-wide frames down; up, the
        valid columns ("kernel": the scatter reads only those) or whole frames ("dma")."""
        down = len(lengths) * self.frame_bytes
        per_token = self.L * 2 * self.H * self.D * 2
        up = sum(lengths) * per_token if self.mode == "kernel" else down
        return down + up

    def close(self):
        torch.cuda.current_stream(self.device).synchronize()
        for arrs in (self.ev_save, self.ev_load, getattr(self, "ev_pack", None)):
            for e in arrs or ():
                e.close()
        self.pinned.close()
