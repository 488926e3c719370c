"""The handoff through pinned host memory: prefill KV -> host frame -> paged cache.

The reference moves every request through host memory: the prefill side pads
each layer group to S columns and downloads it (engines/prefill_full.py:366-384),
the wire carries the S-wide frame (connector/transport.py:29-37, 80-101), and the
decode side uploads and writes it into its cache (engines/decode_batch.py:305-377).
HostStagedHandoff does the same for a batch of requests on one GPU, pipelined
over layers and requests, with nothing synchronising the host between them:

  mode "kernel":
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
  mode "dma" (the default, and the faster one here):
    current stream  per request, one narrow pack into a device frame (all
                    layers), then an event;
    save stream     per request, after its pack: the DMA engine copies the
                    valid columns (K rows up to the 16-token block past P, V
                    rows < P) down into the pinned frame, a few layers per
                    copy, as two rectangular copies (K rows, then V runs)
                    with an event after each;
    load stream     after each of those copies, the same part back up into a
                    second device frame (the other DMA engine);
    current stream  per request, after its last upload: one scatter launch
                    (all layers) into the paged cache;
    host threads    the frames' zero tails (K columns >= round16(P), V rows
                    >= P).
    This is the reference's download / upload shape with copy engines, minus
    the padding: each direction has an engine of its own and no CU is used.

In both modes the pinned frame of a request ends up holding exactly the wire
payload of every layer (K [Hkv, D, S] then V [Hkv, S, D], columns >= P zero),
and the cache holds what pdk_scatter_paged writes from that frame. The caller's
current stream waits for the last scatter, so work issued after run() sees the
cache; run() returns once the host's part is done.

Measured on MI355X: one direction alone moves 53-57 GB/s, by a kernel's
loads or stores through pinned memory or by a DMA engine. Both directions at
once reach about 98 GB/s in total with one DMA engine each way, 77-87 GB/s
with a kernel on either side. On 8 Llama-3.1-8B requests (P uniform in
[64, 512]) "dma" mode takes 6.0 ms (461 MB over the link, 77 GB/s) and
"kernel" mode, whose pack and scatter kernels overlap layer by layer, 9.7 ms
(469 MB, 48 GB/s). Each DMA copy costs about 10 us besides its bytes,
so "dma" mode copies several layers per command (``copy_bytes`` of valid
columns, 16 MiB by default). An upload can start only once its download is
done, so a run takes about the download stream's time plus the longest single
copy: the K and V parts of a chunk are separate copies with an event each,
which halves that copy against one event per chunk.
"""
import ctypes
import os
import threading

import numpy as np
import torch

from .. import _lib
from .._lib import (PDK_COPY_D2H, PDK_COPY_H2D, PDK_EVENT_SYNC, PDK_FRAME_K, PDK_FRAME_V,
                    PDK_PACK_NARROW, PackReq, ScatterReq)
from ..hip import EventArray, PinnedBuffer
from .handoff import _as_layers, _check_cache, _need

MODES = ("kernel", "dma")


class HostStagedHandoff:
    """Pinned host frames for up to ``max_requests`` requests of one model shape."""

    def __init__(self, n_layers, n_kv_heads, head_dim, S, max_requests, device=None,
                 mode="dma", host_threads=None, copy_bytes=16 << 20):
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
            self.ev_read = EventArray(2, PDK_EVENT_SYNC)
        else:
            # Per request: its pack, each of its down copies (at most one K
            # and one V copy per layer), its last up copy; and the run's last
            # up copy.
            self.ev_pack = EventArray(max_requests)
            self.ev_down = EventArray(2 * max_requests * n_layers)
            self.ev_up = EventArray(max_requests)
            self.ev_read = EventArray(2, PDK_EVENT_SYNC)
            shape = (max_requests, n_layers, 2, self.F)
            self.out_frames = torch.empty(shape, dtype=torch.bfloat16, device=self.device)
            self.in_frames = torch.empty(shape, dtype=torch.bfloat16, device=self.device)
        if copy_bytes < 1:
            raise ValueError(f"copy_bytes must be positive, got {copy_bytes}")
        self.copy_bytes = int(copy_bytes)
        self.slot_P = [None] * max_requests
        # Run n records the end of its uploads (kernel mode: of its scatters)
        # in ev_read[n % 2]; run n + 1's host thread waits on that one while
        # the calling thread records ev_read[(n + 1) % 2], so the wait never
        # lands on an event this run has re-recorded.
        self.runs = 0
        self.host_threads = int(host_threads or min(8, os.cpu_count() or 1))
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
            packs.append(self._pack_req(k, v, P, dst, PDK_PACK_NARROW))
            src = self.host_ptr(r) if self.mode == "kernel" else self.in_frames[r].data_ptr()
            scats.append(self._scatter_req(table, P, src))

        def ok(rc, what):
            if rc:
                raise _lib.PdkError(rc, what, _lib.last_error())

        n = len(requests)
        # The zero tails, on host threads, while the device packs and
        # scatters. A slot's new zeros start at its new P: if an earlier,
        # longer request's upload may still read that slot there, wait for
        # the last run's uploads first.
        lengths = [int(P) for _, _, P, _ in requests]
        wait = any(self.slot_P[r] is not None and lengths[r] < self.slot_P[r] for r in range(n))
        prev, slot = (self.runs - 1) % 2, self.runs % 2
        errors = []

        def zero_tails():
            try:
                if wait:                    # a slot with a P is from an earlier run: runs >= 1
                    self.ev_read.sync(prev)
                for r, P in enumerate(lengths):
                    ok(lib.pdk_host_zero_frame_tail(ctypes.c_void_p(self.host_ptr(r)), L, H, D, S,
                                                    P, 64 if kernel else 16, self.host_threads),
                       "pdk_host_zero_frame_tail")
            except BaseException as e:      # re-raised on the calling thread
                errors.append(e)

        filler = threading.Thread(target=zero_tails, name="kv-zero-tails")
        filler.start()
        try:
            self.save_stream.wait_stream(cur)
            self.load_stream.wait_stream(cur)
            if kernel:
                self._run_kernel(lib, ok, packs, scats, cache_k, cache_v, nb, slot)
            else:
                self._run_dma(lib, ok, packs, scats, lengths, cache_k, cache_v, nb, cur, slot)
            cur.wait_stream(self.load_stream)
            cur.wait_stream(self.save_stream)
        finally:
            filler.join()
        if errors:
            raise errors[0]
        for r, P in enumerate(lengths):
            self.slot_P[r] = P
        self.runs += 1

    def _run_kernel(self, lib, ok, packs, scats, cache_k, cache_v, nb, slot):
        # Layer by layer, all requests in one launch each way: 2 L launches
        # for the batch.
        L, S, H, D, n = self.L, self.S, self.H, self.D, len(packs)
        ok(lib.pdk_pack_kv_layerwise((PackReq * n)(*packs), n, L, S, H, D, self.ev_layer.ptr,
                                     self.save_stream.cuda_stream), "pdk_pack_kv_layerwise")
        ok(lib.pdk_scatter_paged_layerwise((ScatterReq * n)(*scats), n, L, S, H, D,
                                           cache_k.data_ptr(), cache_v.data_ptr(),
                                           cache_k.stride(0), nb, self.ev_layer.ptr,
                                           self.load_stream.cuda_stream),
           "pdk_scatter_paged_layerwise")
        ok(lib.pdk_event_record(self.ev_read[slot], self.load_stream.cuda_stream),
           "pdk_event_record")

    def layer_chunks(self, P):
        """(first layer, layers) of each DMA copy of a request of P tokens:
        about ``copy_bytes`` of valid columns per copy, the layers spread
        evenly over the copies. (Copies that start and end a run at one, two
        and four layers do not help: a run takes about the download stream's
        time plus its longest single copy, and they only add copies.)"""
        k1 = min((P + 15) // 16 * 16, self.S)
        per_layer = max(1, (k1 + P) * self.H * self.D * 2)
        n = max(1, min(self.L, self.copy_bytes // per_layer))
        k = -(-self.L // n)               # copies of at most n layers, sizes within one
        out, l0 = [], 0
        for i in range(k):
            m = self.L // k + (1 if i < self.L % k else 0)
            out.append((l0, m))
            l0 += m
        return out

    def _run_dma(self, lib, ok, packs, scats, lengths, cache_k, cache_v, nb, cur, slot):
        L, S, H, D = self.L, self.S, self.H, self.D
        st, save, load = cur.cuda_stream, self.save_stream.cuda_stream, self.load_stream.cuda_stream
        for r, pr in enumerate(packs):
            ok(lib.pdk_pack_kv_batch(ctypes.byref(pr), 1, L, S, H, D, st), "pdk_pack_kv_batch")
            ok(lib.pdk_event_record(self.ev_pack[r], st), "pdk_event_record")
        for r, P in enumerate(lengths):
            out_f, in_f, host = (self.out_frames[r].data_ptr(), self.in_frames[r].data_ptr(),
                                 ctypes.c_void_p(self.host_ptr(r)))
            ok(lib.pdk_stream_wait_event(save, self.ev_pack[r]), "pdk_stream_wait_event")
            for c, (l0, nl) in enumerate(self.layer_chunks(P)):
                for i, part in enumerate((PDK_FRAME_K, PDK_FRAME_V)):
                    ev = self.ev_down[2 * (r * L + c) + i]
                    ok(lib.pdk_copy_frame_valid(host, ctypes.c_void_p(out_f), l0, nl, H, D, S, P,
                                                PDK_COPY_D2H, part, save),
                       "pdk_copy_frame_valid (down)")
                    ok(lib.pdk_event_record(ev, save), "pdk_event_record")
                    ok(lib.pdk_stream_wait_event(load, ev), "pdk_stream_wait_event")
                    ok(lib.pdk_copy_frame_valid(ctypes.c_void_p(in_f), host, l0, nl, H, D, S, P,
                                                PDK_COPY_H2D, part, load),
                       "pdk_copy_frame_valid (up)")
            ok(lib.pdk_event_record(self.ev_up[r], load), "pdk_event_record")
        ok(lib.pdk_event_record(self.ev_read[slot], load), "pdk_event_record")
        for r, sr in enumerate(scats):
            ok(lib.pdk_stream_wait_event(st, self.ev_up[r]), "pdk_stream_wait_event")
            ok(lib.pdk_scatter_paged_batch(ctypes.byref(sr), 1, L, S, H, D, cache_k.data_ptr(),
                                           cache_v.data_ptr(), cache_k.stride(0), nb, st),
               "pdk_scatter_paged_batch")

    def link_bytes(self, lengths):
        """Bytes one run() moves over the host link. "dma" mode: the valid
        columns each way (K rows up to the 16-token block past P, V rows < P).
        "kernel" mode: on the way down the pack's stores (K in whole 64-token
        tiles, V rows < P); on the way up the scatter's loads (columns < P)."""
        half = self.L * self.H * self.D * 2              # one token of K (or V), all layers
        if self.mode == "dma":
            return 2 * sum((min((P + 15) // 16 * 16, self.S) + P) * half for P in lengths)
        down = sum((min((P + 63) // 64 * 64, self.S) + P) * half for P in lengths)
        return down + sum(2 * P * half for P in lengths)

    def close(self):
        torch.cuda.current_stream(self.device).synchronize()
        for name in ("ev_layer", "ev_read", "ev_pack", "ev_down", "ev_up"):
            arr = getattr(self, name, None)
            if arr is not None:
                arr.close()
        self.pinned.close()
