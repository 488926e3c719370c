"""Iteration-level (continuous) decode scheduling onto the paged KV cache.

Follows _ContinuousScheduler (serving/cluster.py:832-1134) and the prefetch of
DecodeWorkerBase (serving/cluster.py:350-436):

* the batch is re-formed before every step: streams whose cache is ready are
  seated in free slots and finished streams leave at once;
* a request's cache is produced in the background when it is submitted
  (PD_KV_LOADERS threads, default 2) and the loop admits only requests whose
  cache is in; a failed load fails that request alone;
* ``admit_min``: with streams running, wait until that many ready requests
  can be taken at once (1 by default);
* occupancy counters: lane-steps, steps, and the empty lanes split into
  starved (nothing was waiting) and held (something waited, admit_min held it);
* a step that raises fails every seated stream and every request taken for
  that iteration, and the loop goes on with a clean batch.

What changes on MI355X is what admission costs. The reference writes a new
stream's whole cache into its lane of a dense [nl, B, ...] tensor
(engines/decode_batch.py:352-377) inside the device lock. Here ``produce``
(run by a loader thread) has already scattered the request's KV into blocks
of the paged cache, so seating a stream is setting up one row of the block
table: nothing is copied under the lock. Decode growth allocates a block every
16 tokens; a finished stream returns its blocks to the free list.

Each step runs the live streams, compacted to the first rows of static
device buffers (tokens, ctx, block tables), through a HIP graph captured once
per batch size, or eagerly with ``use_graphs=False``.
"""
import collections
import os
import threading
import time
from concurrent.futures import ThreadPoolExecutor

import torch


class ContinuousScheduler:
    """Continuous batching of up to ``B`` streams over one decoder and paged cache.

    decoder: engines.llama_decode.LlamaDecoder (or an object with its step /
      capture interface); cache: engines.paged_cache.PagedKVCache.
    produce(item) -> (first_token, pos, aux_ms): makes the request's KV resident
      in ``cache`` under item["req_id"] (tokens 0..pos-1), returning the first
      token to decode and its position (the prompt length).
    Items are dicts with "req_id" and "max_new" (tokens to return, the first
    included); an ``on_token(item, tok)`` callback streams them.
    """

    def __init__(self, B, decoder, cache, produce, admit_min=1, loaders=None, max_blocks=None,
                 use_graphs=True, on_token=None, device=None):
        self.B, self.dec, self.cache, self.produce = B, decoder, cache, produce
        self.admit_min = admit_min
        self.on_token = on_token
        self.use_graphs = use_graphs
        self.device = torch.device(device) if device else cache.k.device
        n = loaders if loaders is not None else int(os.environ.get("PD_KV_LOADERS", "2"))
        self._loader = ThreadPoolExecutor(max_workers=max(1, n))
        self.max_blocks = max_blocks or 64                   # table width: 1024 tokens per stream
        self.slots = [None] * B
        self.pending = collections.deque()
        self.cv = threading.Condition()
        self.admit_ms, self.admits = 0.0, 0
        self.lane_steps, self.steps = 0, 0
        self.starved_lane_steps = 0
        self.held_lane_steps = 0
        self.admit_stall_ms = 0.0
        # (start on the monotonic clock, duration ms, streams) of each step
        # since the last take_step_log(): what a serving run correlates with
        # other processes' work on the same GPU. The loop appends and
        # take_step_log swaps under _log_lock, so no step is lost in between.
        self.step_log = []
        self._log_lock = threading.Lock()
        # Step inputs: one pinned host block and its device copy, as int32
        # [tokens B | ctx B | tables B x max_blocks]; the step reads views of
        # the device copy, so a captured graph sees each step's values.
        self._width = 2 * B + B * self.max_blocks
        self._host = torch.zeros(self._width, dtype=torch.int32,
                                 pin_memory=self.device.type == "cuda")
        self._dev = torch.zeros(self._width, dtype=torch.int32, device=self.device)
        self._graphs = {}
        # Decode runs on a stream of its own: loader threads order their
        # scatters after their thread's current stream, which must not be
        # the one holding queued decode steps. A loaded request is seated
        # only after its loader synchronised, so decode sees its blocks.
        self.stream = torch.cuda.Stream(self.device) if self.device.type == "cuda" else None
        self._stop = False
        self._thread = threading.Thread(target=self._loop, daemon=True)
        self._thread.start()

    def _on_stream(self):
        import contextlib
        return torch.cuda.stream(self.stream) if self.stream is not None else contextlib.nullcontext()

    def warmup(self):
        """Capture the step graph of every batch size 1..B before serving.

        Each capture runs one real step first; here every row decodes token 0
        at position 0 of block 0, which no request owns yet (the cache must be
        empty), and whoever gets block 0 later overwrites it whole."""
        if not self.use_graphs:
            return
        if self._active() or self.pending or \
                self.cache.alloc.free_blocks() != self.cache.num_blocks:
            raise RuntimeError("warmup needs an idle scheduler and an empty cache")
        B, mb = self.B, self.max_blocks
        self.dec.reserve(mb * 16)
        host = self._host.numpy()
        host[:] = 0
        host[B:2 * B] = 1
        tables = host[2 * B:].reshape(B, mb)
        tables[:] = -1
        tables[:, 0] = 0
        with self._on_stream():
            self._dev.copy_(self._host)
            tab = self._dev[2 * B:].view(B, mb)
            for b in range(1, B + 1):
                if b not in self._graphs:
                    self._graphs[b] = self.dec.capture(self._dev[:b], self._dev[B:B + b],
                                                       tab[:b], mb * 16)
        torch.cuda.synchronize(self.device)

    # -- requests ---------------------------------------------------------------
    def submit_async(self, item):
        """Queue a request and start its cache load; returns the item (its
        "ev" is set when it finishes, with "out" or "err")."""
        item["ev"] = threading.Event()
        item["out"] = item["err"] = None
        item["_fut"] = self._loader.submit(self.produce, item)
        item["_fut"].add_done_callback(lambda _f: self._wake())
        with self.cv:
            self.pending.append(item)
            self.cv.notify()
        return item

    def submit(self, item):
        """Queue a request and block until it finishes (the reference's submit)."""
        self.submit_async(item)
        item["ev"].wait()
        if item["err"]:
            raise item["err"]
        return item["out"]

    def close(self):
        with self.cv:
            self._stop = True
            self.cv.notify()
        self._thread.join(timeout=10)
        self._loader.shutdown(wait=True)

    def take_step_log(self):
        """The steps since the last call: [(start s, duration ms, streams)]."""
        with self._log_lock:
            log, self.step_log = self.step_log, []
        return log

    def _active(self):
        return [s for s in self.slots if s]

    def _wake(self):
        with self.cv:
            self.cv.notify()

    def _ready_pending(self):
        """Move finished loads to the front; fail the requests whose load failed.
        Called with self.cv held."""
        keep, ready = collections.deque(), []
        for item in self.pending:
            fut = item["_fut"]
            if not fut.done():
                keep.append(item)
            elif fut.exception() is not None:
                item["err"] = fut.exception()                # this request only
                self._release(item)
                item["ev"].set()
            else:
                first, pos, aux_ms = fut.result()
                if pos + item["max_new"] > self.max_blocks * 16:
                    item["err"] = ValueError(
                        f"{item['req_id']}: {pos} + {item['max_new']} tokens exceed the block "
                        f"table width of {self.max_blocks * 16} tokens")
                    self._release(item)
                    item["ev"].set()
                    continue
                item["_produced"] = (first, pos, aux_ms)
                ready.append(item)
        self.pending = collections.deque(ready + list(keep))
        return len(ready)

    def _release(self, item):
        try:
            self.cache.free(item["req_id"])
        except Exception:
            pass

    # -- seating and finishing ----------------------------------------------------
    def _seat(self, idx, item):
        first, pos, aux_ms = item.pop("_produced")
        item["first"], item["pos"] = first, pos
        self.slots[idx] = {"item": item, "cur": first, "pos": pos, "pos0": pos,
                           "s0": self.steps, "l0": self.lane_steps,
                           "v0": self.starved_lane_steps, "h0": self.held_lane_steps,
                           "outs": [first], "load_ms": aux_ms, "steps": [],
                           "t0": time.perf_counter()}
        self._emit(item, first)
        if item["max_new"] <= 1:
            self._finish(idx)

    def _emit(self, item, tok):
        if self.on_token is not None:
            self.on_token(item, tok)

    def _finish(self, idx):
        s, self.slots[idx] = self.slots[idx], None
        st = sorted(s["steps"])
        dsteps = max(self.steps - s["s0"], 1)
        win = lambda now, then: (now - then) / dsteps   # noqa: E731
        s["item"]["out"] = {
            "tokens": s["outs"], "load_ms": round(s["load_ms"], 1),
            "prefill_ms": round(s["load_ms"], 1), "pos": s["pos0"],
            "tpot_ms": round(st[len(st) // 2], 3) if st else 0.0,
            "decode_ms": round((time.perf_counter() - s["t0"]) * 1e3, 1),
            "batch": len(self._active()) + 1, "batch_width": self.B, "sched": "continuous",
            "admit_ms": round(self.admit_ms / max(self.admits, 1), 3),
            "occupancy": round(win(self.lane_steps, s["l0"]), 2),
            "starved_lanes": round(win(self.starved_lane_steps, s["v0"]), 2),
            "held_lanes": round(win(self.held_lane_steps, s["h0"]), 2),
            "occupancy_all": round(self.lane_steps / max(self.steps, 1), 2),
            "admit_stall_ms": round(self.admit_stall_ms, 3)}
        self._release(s["item"])
        s["item"]["ev"].set()

    # -- one decode step ------------------------------------------------------------
    def _step(self, live):
        """Run one step for the seated streams ``live`` (slot indices); returns
        the next token per stream."""
        b, mb, B = len(live), self.max_blocks, self.B
        host = self._host.numpy()
        host[:] = 0
        tables = host[2 * B:].reshape(B, mb)
        tables[:b] = -1
        for row, i in enumerate(live):
            s = self.slots[i]
            req = s["item"]["req_id"]
            self.cache.ensure(req, s["pos"] + 1)                 # a new block every 16 tokens
            blocks = self.cache.blocks(req)
            host[row] = s["cur"]
            host[B + row] = s["pos"] + 1
            tables[row, :len(blocks)] = blocks
        self._dev.copy_(self._host, non_blocking=True)
        tok, ctx = self._dev[:b], self._dev[B:B + b]
        tab = self._dev[2 * B:].view(B, mb)[:b]
        if self.use_graphs:
            g = self._graphs.get(b)
            if g is None:
                self.dec.reserve(mb * 16)
                # Capture runs one eager step first: it is this step.
                g = self._graphs[b] = self.dec.capture(tok, ctx, tab, mb * 16)
            else:
                g.replay()
        else:
            self.dec.step(tok, ctx, tab, mb * 16)
        return self.dec.tokens[:b].cpu().tolist()

    def _loop(self):
        while True:
            with self.cv:
                while True:
                    if self._stop:
                        return
                    ready = self._ready_pending()
                    if ready or self._active():
                        break
                    self.cv.wait(timeout=None if not self.pending else 0.05)
                free = [i for i, s in enumerate(self.slots) if s is None]
                n = min(len(free), ready)
                if n and not self._active():
                    pass                                 # idle: take whatever is ready
                elif n < min(self.admit_min, len(free)):
                    n = 0
                taking = [(free[k], self.pending.popleft()) for k in range(n)]
                self.starved_lane_steps += len(free) - min(len(free), len(self.pending) + n)
                self.held_lane_steps += (len(free) - n) - max(
                    0, len(free) - len(self.pending) - n)
            try:
                if taking:
                    t0 = time.perf_counter()
                    for idx, item in taking:
                        self._seat(idx, item)
                    ms = (time.perf_counter() - t0) * 1e3
                    self.admit_ms += ms
                    self.admit_stall_ms += ms
                    self.admits += 1
                live = [i for i, s in enumerate(self.slots) if s]
                if not live:
                    continue
                t_mono = time.monotonic()
                t1 = time.perf_counter()
                with self._on_stream():
                    nxt = self._step(live)
                dt = (time.perf_counter() - t1) * 1e3
                self.lane_steps += len(live)
                self.steps += 1
                with self._log_lock:
                    if len(self.step_log) < 1_000_000:
                        self.step_log.append((t_mono, dt, len(live)))
                for row, i in enumerate(live):
                    s = self.slots[i]
                    s["steps"].append(dt)
                    s["outs"].append(nxt[row])
                    self._emit(s["item"], nxt[row])
                    s["cur"] = nxt[row]
                    s["pos"] += 1
                    if len(s["outs"]) >= s["item"]["max_new"]:
                        self._finish(i)
            except Exception as e:                       # a bad step fails its batch
                for i, s in enumerate(self.slots):
                    if s:
                        s["item"]["err"] = e
                        self._release(s["item"])
                        s["item"]["ev"].set()
                        self.slots[i] = None
                for _idx, item in taking:
                    if not item["ev"].is_set():
                        item["err"] = item.get("err") or e
                        self._release(item)
                        item["ev"].set()


class Prefetcher:
    """Start a request's cache load before its decode request arrives
    (DecodeWorkerBase.prefetch / _load_kv, serving/cluster.py:350-436).

    At most ``cap`` loads are held (PD_PREFETCH_CAP, 8); a new request is
    skipped when full rather than dropping a live entry, whose load has already
    taken the request's KV out of the transport; entries older than ``ttl_s``
    (PD_PREFETCH_TTL_S, 900) belong to abandoned requests and are reclaimed."""

    def __init__(self, load, cap=None, ttl_s=None):
        self.load = load
        self.cap = cap if cap is not None else int(os.environ.get("PD_PREFETCH_CAP", "8"))
        self.ttl_s = ttl_s if ttl_s is not None else float(os.environ.get("PD_PREFETCH_TTL_S", "900"))
        self._jobs = {}
        self._lock = threading.Lock()

    def prefetch(self, req_id):
        with self._lock:
            if req_id in self._jobs:
                return {"prefetch": "already running"}
            now = time.perf_counter()
            for old in [k for k, (_p, _f, t) in self._jobs.items() if now - t > self.ttl_s]:
                pool, _fut, _t0 = self._jobs.pop(old)
                pool.shutdown(wait=False)
            if len(self._jobs) >= self.cap:
                return {"prefetch": "skipped (full)", "req_id": req_id}
            pool = ThreadPoolExecutor(max_workers=1)
            self._jobs[req_id] = (pool, pool.submit(self.load, req_id), time.perf_counter())
        return {"prefetch": "started", "req_id": req_id}

    def take(self, req_id):
        """(result, lead_ms) of a prefetch, joining it if still running; a fresh
        load (lead_ms -1) when none was started."""
        with self._lock:
            entry = self._jobs.pop(req_id, None)
        if entry is None:
            return self.load(req_id), -1.0
        pool, fut, t0 = entry
        try:
            res = fut.result()
            return res, (time.perf_counter() - t0) * 1e3
        finally:
            pool.shutdown(wait=False)

    def outstanding(self):
        with self._lock:
            return list(self._jobs)


__all__ = ["ContinuousScheduler", "Prefetcher"]
