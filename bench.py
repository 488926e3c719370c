#!/usr/bin/env python3
"""Benchmark of the prefill->decode KV handoff and decode_batch attention on one MI355X.

Metric (one JSON line on stdout): KV handoff GB/s over a batch of 8 Llama-3.1-8B
requests (32 layers x K/V x 8 KV heads x head_dim 128, bf16, S=512 frames,
lengths uniform in [64, 512] from seed 0), with the ms per 512-token request and
decode_batch tokens/s alongside.

  handoff   (the value) the batch staged through pinned host memory as a
            pipeline across requests ("dma" mode): each request is packed
            narrow (valid columns) into a device frame; the DMA engines copy
            its valid columns down into its pinned S-wide wire frame, a few
            layers per copy, on a save stream and back up into a second device
            frame on a load stream; host threads write the frames' zero tails;
            one scatter per request places the frame in the paged decode cache
            (block 16, seeded permuted block table). A step is one batch;
            handoff bytes = sum(P) * 131072 B. The step is bound by the host
            link (value_bound: its link bytes per second against this run's
            both-ways DMA rate); its own kernels are timed under kernels.
            Beside it: the device-only S-wide pack and scatter of the batch
            (the HBM-bound kernels; roofline is that pack), the same staging
            with the kernels' own loads and stores through pinned memory
            ("kernel" mode), one 512-token request, KONI token blocks and the
            host-link rates.
  shm       the drop-in shm transport on the device path: RngdKVConnector on
            select_transport("shm"), device save -> /dev/shm -> device load
            into the paged cache, for one 512-token request and for the batch.
  decode    GQA decode attention, 32 layers x B streams at context 512, per-layer
            launches, eager and replayed from a HIP graph; B=16 at context 2048
            (one context split, no merge launch) from a graph.
  step      the full Llama-3.1-8B decode step (random-init weights) at B=4 and
            B=16, context 512, eager and from a HIP graph, beside the
            reference's published 21.54 / 35.54 ms per step.
  serve     2 prefill producers + 1 decode consumer on this GPU:
            64 requests, Poisson(20/s), prompts U[128,1024], 128 greedy tokens.
  cpu       the oracle's restatement of the reference CPU shm path (ser -> /dev/shm
            -> deser -> f32 place) on a bounded sample of the same requests.

  python bench.py [--steps K] [--warmup W] [--cpu-seconds X]
"""
import argparse
import ctypes
import gc
import json
import math
import os
import shutil
import statistics
import sys
import tempfile
import time

import numpy as np

L, H, D, S, BS = 32, 8, 128, 512, 16
HQ = 32
TOKEN_BYTES = L * 2 * H * D * 2          # 131072 B of K+V per token, all layers
HBM_PEAK_GBS = 8000.0
METRIC = "KV handoff GB/s + ms per 512-tok Llama-8B request; decode_batch tokens/s"


def parse():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--cpu-seconds", type=float, default=12.0,
                    help="bound on the CPU baseline sample (0 skips it)")
    ap.add_argument("--only", default="all",
                    help="restrict the run (for profiler passes): all, or a comma-separated "
                         "subset of handoff, shm, decode, step, long, serve, copy")
    ap.add_argument("--copy-mib", type=int, default=1024,
                    help="bytes moved by --only copy (traffic-counter calibration)")
    args = ap.parse_args()
    legs = {"all", "handoff", "shm", "decode", "step", "long", "serve", "copy"}
    args.legs = set(args.only.split(","))
    if not args.legs <= legs:
        ap.error(f"--only: unknown legs {sorted(args.legs - legs)}")
    return args


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def measured_traffic(kernel):
    """HBM bytes per launch of ``kernel`` from the committed rocprofv3 --pmc summary
    (FETCH_SIZE and WRITE_SIZE, scaled by the copy-kernel calibration), or None."""
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", "traffic.json")
    try:
        with open(path) as f:
            t = json.load(f)
    except (OSError, ValueError):
        return None
    k, c = t.get("kernels", {}).get(kernel), t.get("calibration", {})
    if not k:
        return None
    return int((k["fetch_kib"] * c["fetch_scale"] + k["write_kib"] * c["write_scale"]) * 1024)


def roofline(bytes_per_launch, seconds_per_launch, traffic=None):
    achieved = bytes_per_launch / seconds_per_launch / 1e9
    return {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic,
            "bytes_per_launch": int(bytes_per_launch),
            "us_per_launch": round(seconds_per_launch * 1e6, 2)}


class Timer:
    """HIP-event pairs on torch's current stream (the stream the kernels run on).

    The events are created up front, `n` intervals per timer: a host stall between
    a begin and an end (an event created or a collection run inside the loop)
    lands inside the measured interval, and one such stall of a few tens of
    milliseconds in 50 steps would add several hundred microseconds to a mean."""

    def __init__(self, torch, n=256):
        self.torch = torch
        self.pool = [torch.cuda.Event(enable_timing=True) for _ in range(2 * n)]
        for e in self.pool:          # torch creates the HIP event at its first record
            e.record()
        torch.cuda.synchronize()
        self.used = 0
        self.pairs = {}

    def _event(self):
        if self.used == len(self.pool):
            raise RuntimeError("Timer: more intervals than reserved")
        e = self.pool[self.used]
        self.used += 1
        e.record()
        return e

    def begin(self, name):
        self.pairs.setdefault(name, []).append([self._event(), None])

    def end(self, name):
        self.pairs[name][-1][1] = self._event()

    def mean_s(self, name):
        ms = [a.elapsed_time(b) for a, b in self.pairs[name]]
        return statistics.fmean(ms) / 1e3

    def median_s(self, name):
        return statistics.median(a.elapsed_time(b) for a, b in self.pairs[name]) / 1e3


def gpu_delay(torch, us):
    """A function that queues a bounded spin of about `us` microseconds on torch's
    current stream (torch.cuda._sleep, calibrated once with HIP events). Queued
    before a batch of short launches, it lets the host enqueue all of them before
    the first one starts, so events around the batch time the kernels back to
    back rather than the host's launch rate. Without torch.cuda._sleep the
    function queues nothing (and the times may then include host gaps)."""
    if not hasattr(torch.cuda, "_sleep"):
        return lambda: None
    probe = 1 << 20
    t = Timer(torch, 1)
    t.begin("spin")
    torch.cuda._sleep(probe)
    t.end("spin")
    torch.cuda.synchronize()
    cycles = max(1, int(probe * us * 1e-6 / t.mean_s("spin")))
    return lambda: torch.cuda._sleep(cycles)


def workload(seed=0, n=8):
    rng = np.random.default_rng(seed)
    return [int(p) for p in rng.integers(64, S + 1, n)]


def make_tables(torch, dev, lengths, seed=0, slack=16):
    rng = np.random.default_rng(seed + 1)
    need = [(p + BS - 1) // BS for p in lengths]
    nb = sum(need) + slack
    perm = rng.permutation(nb).astype(np.int32)
    tables, off = [], 0
    for n in need:
        tables.append(torch.from_numpy(perm[off:off + n].copy()).to(dev))
        off += n
    return nb, tables


def bench_handoff(args, torch, K, lib, dev, out):
    """The headline: the 8-request batch staged through pinned host
    memory, pipelined across requests and layers with no host synchronisation
    between them (HostStagedHandoff, "dma" mode: narrow pack into device
    frames; the DMA engines copy each request's valid columns down into its
    pinned S-wide frame, a few layers per copy, and back up into a second
    device frame on another stream; host threads write the frames' zero tails;
    one scatter per request into the paged cache). A step is one such batch;
    value = handoff bytes (sum P * 131072) per second of wall time over the K
    timed steps.

    Beside it: the device-only pack and scatter kernels on the same batch (the
    HBM-bound kernels, whose rooflines are reported), the "kernel" staging
    mode (the kernels' own loads and stores through pinned memory), one
    512-token request each way, the same request as KONI token blocks, and the
    host-link rates."""
    from rngd_pd_amd._lib import PackReq, ScatterReq
    from rngd_pd_amd.kernels.staging import HostStagedHandoff
    lengths = workload()
    n = len(lengths)
    gen = torch.Generator(device=dev).manual_seed(0)
    prefill = [torch.randn((L, 2, S, H, D), generator=gen, device=dev).to(torch.bfloat16)
               for _ in lengths]
    frames = [torch.empty(K.frame_shape(L, H, D, S), dtype=torch.bfloat16, device=dev)
              for _ in lengths]
    nb, tables = make_tables(torch, dev, lengths)
    cache_k = torch.zeros((L, nb, H, BS, D), dtype=torch.bfloat16, device=dev)
    cache_v = torch.zeros((L, nb, H, D, BS), dtype=torch.bfloat16, device=dev)
    tokens = sum(lengths)
    handoff_bytes = tokens * TOKEN_BYTES

    # -- the device-only kernels on the batch (HBM roofline) -------------------
    pack = (PackReq * n)(*[
        PackReq(p.data_ptr(), p[:, 1].data_ptr(), f.data_ptr(), p.stride(0), p.stride(2), P, 0)
        for p, f, P in zip(prefill, frames, lengths)])
    scat = (ScatterReq * n)(*[
        ScatterReq(f.data_ptr(), t.data_ptr(), P, t.numel())
        for f, t, P in zip(frames, tables, lengths)])
    st = torch.cuda.current_stream().cuda_stream

    def device_step(timer=None):
        if timer:
            timer.begin("pack")
        rc = lib.pdk_pack_kv_batch(pack, n, L, S, H, D, st)
        if rc:
            raise RuntimeError("pack launch failed: " + lib.pdk_last_error().decode())
        if timer:
            timer.end("pack")
            timer.begin("scatter")
        rc = lib.pdk_scatter_paged_batch(scat, n, L, S, H, D, cache_k.data_ptr(),
                                         cache_v.data_ptr(), cache_k.stride(0), nb, st)
        if rc:
            raise RuntimeError("scatter launch failed: " + lib.pdk_last_error().decode())
        if timer:
            timer.end("scatter")

    for _ in range(args.warmup):
        device_step()
    torch.cuda.synchronize()
    # Spot check of the kernels: request 0 gathered back equals its packed frame.
    back = K.gather_paged(cache_k, cache_v, tables[0], lengths[0], S)
    torch.cuda.synchronize()
    if not torch.equal(back.view(torch.int16), frames[0].view(torch.int16)):
        raise RuntimeError("device handoff round trip is not bit-exact")
    timer = Timer(torch, 4 * args.steps)
    t0 = time.perf_counter()
    for _ in range(args.steps):
        device_step(timer)
    torch.cuda.synchronize()
    dev_wall = (time.perf_counter() - t0) / args.steps
    pack_bytes = (tokens + n * S) * TOKEN_BYTES       # read valid tokens + write S-wide frames
    scat_bytes = 2 * tokens * TOKEN_BYTES             # read valid frame columns + write blocks
    out["roofline"] = dict(roofline(pack_bytes, timer.mean_s("pack"),
                                    measured_traffic("pack_kv_batch")),
                           kernel="pack_kv_batch: the 8 requests' S-wide frames in one launch, "
                                  "device-only (HBM-bound); the timed step is host-link-bound "
                                  "(value_bound) and its own kernels are under kernels")
    out["kernels"] = {"pack_kv_batch": out["roofline"],
                      "scatter_paged_batch": roofline(scat_bytes, timer.mean_s("scatter"),
                                                      measured_traffic("scatter_paged_batch"))}
    out["extra"]["device_batch"] = {
        "gbps": round(handoff_bytes / dev_wall / 1e9, 1), "ms": round(dev_wall * 1e3, 4),
        "what": "pack + scatter of the batch with prefill KV resident in HBM, no host staging"}
    log(f"device batch: {handoff_bytes / dev_wall / 1e9:.1f} GB/s, pack "
        f"{timer.mean_s('pack') * 1e6:.1f} us, scatter {timer.mean_s('scatter') * 1e6:.1f} us")
    ref_k, ref_v = cache_k.clone(), cache_v.clone()

    # -- the kernels the staged step itself runs -------------------------------
    # The dma-mode step packs each request narrow (valid columns only) into a
    # device frame and scatters each request from its uploaded frame: 8
    # launches of each per step, timed here on device frames as one group per
    # kind (events around the 8 launches, mean per launch), queued behind a
    # spin so that the host's launch rate does not enter the times.
    from rngd_pd_amd._lib import PDK_PACK_NARROW
    narrow = [PackReq(p.data_ptr(), p[:, 1].data_ptr(), f.data_ptr(), p.stride(0), p.stride(2),
                      P, PDK_PACK_NARROW) for p, f, P in zip(prefill, frames, lengths)]
    timer_n = Timer(torch, 4 * args.steps)
    delay = gpu_delay(torch, 1000)
    for i in range(args.warmup + args.steps):
        if i >= args.warmup:
            delay()
            timer_n.begin("pack")
        for r in range(n):
            if lib.pdk_pack_kv_batch(ctypes.byref(narrow[r]), 1, L, S, H, D, st):
                raise RuntimeError("narrow pack failed: " + lib.pdk_last_error().decode())
        if i >= args.warmup:
            timer_n.end("pack")
            timer_n.begin("scatter")
        for r in range(n):
            if lib.pdk_scatter_paged_batch(ctypes.byref(scat[r]), 1, L, S, H, D,
                                           cache_k.data_ptr(), cache_v.data_ptr(),
                                           cache_k.stride(0), nb, st):
                raise RuntimeError("scatter failed: " + lib.pdk_last_error().decode())
        if i >= args.warmup:
            timer_n.end("scatter")
    torch.cuda.synchronize()
    half = L * H * D * 2                                # one token of K (or V), all layers
    narrow_bytes = sum(P * TOKEN_BYTES + (min((P + 63) // 64 * 64, S) + P) * half
                       for P in lengths) / n
    scat_req_bytes = scat_bytes / n
    out["kernels"]["pack_kv_narrow_per_request"] = dict(
        roofline(narrow_bytes, timer_n.mean_s("pack") / n),
        what="pack_kernel on one request into a device frame, valid columns only (the staged "
             "step's pack); mean per launch over the batch's 8 requests")
    out["kernels"]["scatter_paged_per_request"] = dict(
        roofline(scat_req_bytes, timer_n.mean_s("scatter") / n),
        what="scatter_kernel of one request (the staged step's scatter); mean per launch")
    log(f"staged step's kernels: narrow pack {timer_n.mean_s('pack') / n * 1e6:.1f} us, "
        f"scatter {timer_n.mean_s('scatter') / n * 1e6:.1f} us per request")
    torch.cuda.synchronize()
    if not (torch.equal(cache_k.view(torch.int16), ref_k.view(torch.int16))
            and torch.equal(cache_v.view(torch.int16), ref_v.view(torch.int16))):
        raise RuntimeError("per-request scatters differ from the batched scatter")
    # The narrow packs left the frames' tails as they were (the S-wide pack
    # wrote zeros there); restore the S-wide frames for the checks below.
    if lib.pdk_pack_kv_batch(pack, n, L, S, H, D, st):
        raise RuntimeError("pack launch failed: " + lib.pdk_last_error().decode())
    torch.cuda.synchronize()

    # -- the batch staged through pinned host memory (value) -----------------
    reqs = [(p[:, 0], p[:, 1], P, t) for p, P, t in zip(prefill, lengths, tables)]
    staged = {}
    for mode in ("dma", "kernel"):
        stager = HostStagedHandoff(L, H, D, S, n, device=dev, mode=mode)
        cache_k.zero_()
        cache_v.zero_()
        steps = args.steps if mode == "dma" else max(3, min(args.steps, 10))
        for _ in range(max(1, args.warmup)):
            stager.run(reqs, cache_k, cache_v)
        torch.cuda.synchronize()
        # The timed path's result: the cache equals the device kernels' result,
        # and each pinned frame is that request's S-wide wire payload.
        if not (torch.equal(cache_k.view(torch.int16), ref_k.view(torch.int16))
                and torch.equal(cache_v.view(torch.int16), ref_v.view(torch.int16))):
            raise RuntimeError(f"staged ({mode}) cache differs from the device kernels' cache")
        for r in range(n):
            host = torch.from_numpy(stager.host_frame(r).view(np.int16))
            if not torch.equal(host.view(-1), frames[r].view(torch.int16).cpu().view(-1)):
                raise RuntimeError(f"staged ({mode}) host frame {r} differs from the packed frame")
        t0 = time.perf_counter()
        for _ in range(steps):
            stager.run(reqs, cache_k, cache_v)
        torch.cuda.synchronize()
        wall = (time.perf_counter() - t0) / steps
        link = stager.link_bytes(lengths)
        staged[mode] = {"gbps": round(handoff_bytes / wall / 1e9, 2), "ms": round(wall * 1e3, 3),
                        "steps": steps, "host_link_bytes": link,
                        "host_link_gbps": round(link / wall / 1e9, 1)}
        if mode == "dma":
            out["value"] = staged[mode]["gbps"]
            out["ms_per_step"] = staged[mode]["ms"]
        log(f"staged batch ({mode}): {staged[mode]['gbps']} GB/s, {staged[mode]['ms']} ms, "
            f"host link {staged[mode]['host_link_gbps']} GB/s")
        stager.close()
    out["extra"]["staged_batch"] = staged
    out["config"]["lengths"] = lengths
    out["config"]["handoff_bytes_per_step"] = handoff_bytes

    # -- one 512-token request: device path, and staged each way --------------
    p512 = prefill[0]
    f512 = frames[0]
    nb1 = (S + BS - 1) // BS
    t512 = torch.from_numpy(np.random.default_rng(5).permutation(nb).astype(np.int32)[:nb1]).to(dev)
    single = Timer(torch, 4 * args.steps)
    for i in range(args.warmup + args.steps):
        if i >= args.warmup:
            single.begin("req")
        K.pack_kv(p512[:, 0], p512[:, 1], S, S, frame=f512)
        K.scatter_paged(f512, t512, S, S, cache_k, cache_v)
        if i >= args.warmup:
            single.end("req")
    torch.cuda.synchronize()
    out["extra"]["ms_per_512_request_device"] = round(single.median_s("req") * 1e3, 4)
    out["extra"]["gbps_512_request_device"] = round(S * TOKEN_BYTES / single.median_s("req") / 1e9, 1)
    one = [(p512[:, 0], p512[:, 1], S, t512)]
    for mode in ("dma", "kernel"):
        stager = HostStagedHandoff(L, H, D, S, 1, device=dev, mode=mode)
        ms = []
        for i in range(max(1, args.warmup) + max(5, min(args.steps, 20))):
            torch.cuda.synchronize()
            a = time.perf_counter()
            stager.run(one, cache_k, cache_v)
            torch.cuda.synchronize()
            if i >= max(1, args.warmup):
                ms.append((time.perf_counter() - a) * 1e3)
        stager.close()
        out["extra"][f"ms_per_512_request_staged_{mode}"] = round(statistics.median(ms), 3)
    best = out["extra"]["ms_per_512_request_staged_dma"]      # the default mode
    out["extra"]["ms_per_512_request_staged"] = best
    out["extra"]["gbps_512_request_staged"] = round(S * TOKEN_BYTES / best / 1e6, 2)
    log(f"512-token request: device {out['extra']['ms_per_512_request_device']} ms, staged "
        f"kernel {out['extra']['ms_per_512_request_staged_kernel']} ms, dma "
        f"{out['extra']['ms_per_512_request_staged_dma']} ms")

    # -- the same request as KONI token blocks ---------------------------------
    # Prefill KV [L][2][S][Hkv][D] is already the Furiosa native wire's units in
    # order (unit (2l + kind) * S + token), so placement reads it in place.
    koni = Timer(torch, 4 * args.steps)
    index = torch.arange(2 * L * S, dtype=torch.int32, device=dev).view(2 * L, S)
    for i in range(args.warmup + args.steps):
        if i >= args.warmup:
            koni.begin("req")
        rc = lib.pdk_scatter_koni(p512.data_ptr(), 2 * L * S, index.data_ptr(), 2 * L, S,
                                  t512.data_ptr(), t512.numel(), cache_k.data_ptr(),
                                  cache_v.data_ptr(), cache_k.stride(0), nb, H, D,
                                  torch.cuda.current_stream().cuda_stream)
        if i >= args.warmup:
            koni.end("req")
        if rc:
            raise RuntimeError("koni scatter failed: " + lib.pdk_last_error().decode())
    torch.cuda.synchronize()
    kt = koni.median_s("req")
    out["extra"]["koni_512_request"] = {
        "us": round(kt * 1e6, 2), "roofline": roofline(2 * S * TOKEN_BYTES, kt)}

    bench_host_link(args, torch, lib, dev, out, frames[0])
    both = out["extra"]["host_link"]["dma_both_ways_total_gbps"]
    for mode, row in staged.items():
        row["host_link_frac_of_dma_both_ways"] = round(row["host_link_gbps"] / both, 3)
    # What bounds the timed step: the host link, both directions at once.
    dma = staged["dma"]
    out["value_bound"] = {
        "bound": "host link", "unit": "GB/s",
        "link_bytes_per_step": dma["host_link_bytes"], "achieved": dma["host_link_gbps"],
        "ceiling": both, "ceiling_what": "64 MiB DMA copies down and up at once, this run",
        "frac": dma["host_link_frac_of_dma_both_ways"],
        "kernels": "pack_kv_narrow_per_request, scatter_paged_per_request (under kernels)"}


def bench_shm(args, torch, K, dev, out):
    """The drop-in shm transport on the device path, timed per request as the
    reference times its shm handoff (bench/nixl_kv_check.py:211-221: save,
    download, load of one request): RngdKVConnector on
    select_transport("shm"), device save (pack on a side stream, pinned
    staging, one ordered writer: tmp + fsync + rename per blob) -> /dev/shm
    files (the reference's wire, byte for byte) -> device load (read into
    pinned memory, copy up, scatter into the paged cache, files consumed).
    One 512-token Llama-3.1-8B request (64 MiB on the wire), then the 8
    requests of the handoff batch saved one after the other and loaded one
    after the other. The files' payloads and the loaded cache are checked
    against the device pack once, outside the timed loops."""
    from rngd_pd_amd.connector import transport as kvt
    from rngd_pd_amd.connector.rngd_kv import KVConnectorRole, RngdKVConnector
    from rngd_pd_amd.connector.wire import decode_payload
    from rngd_pd_amd.engines.paged_cache import PagedKVCache
    lengths = workload()
    gen = torch.Generator(device=dev).manual_seed(0)
    prefill = [torch.randn((L, 2, S, H, D), generator=gen, device=dev).to(torch.bfloat16)
               for _ in lengths]
    root = tempfile.mkdtemp(prefix="pd-shm-bench-", dir="/dev/shm" if os.path.isdir("/dev/shm")
                            else None)
    saved_env = {k: os.environ.get(k) for k in ("PD_SHM_ROOT", "AIRM_KV_TRANSPORT")}
    os.environ["PD_SHM_ROOT"], os.environ["AIRM_KV_TRANSPORT"] = root, "shm"
    kvt.reset_selection()
    per = (S + BS - 1) // BS
    cache = PagedKVCache(L, per * (len(lengths) + 1), H, D, device=dev)

    def save(req, p, P):
        c = RngdKVConnector(KVConnectorRole.WORKER, req_id=req, n_layers=L, frame_tokens=S)
        for i in range(L):
            c.save_kv_layer(f"layer.{i}", (p[i, 0], p[i, 1]), num_tokens=P)
        c.wait_for_save()
        c.close()

    def load(req, P):
        c = RngdKVConnector(KVConnectorRole.WORKER, req_id=req, n_layers=L)
        c.register_kv_caches(cache.view(req, P, S))
        c.start_load_kv()
        for i in range(L):
            c.wait_for_layer_load(f"layer.{i}")
        c.close()
        torch.cuda.synchronize()

    try:
        # Check: request 0's files hold the packed frame's bytes, and the
        # load places exactly that frame.
        P0 = lengths[0]
        frame = K.pack_kv(prefill[0][:, 0], prefill[0][:, 1], P0, S)
        torch.cuda.synchronize()
        want = frame.view(torch.int16).cpu().numpy().view(np.uint16).reshape(L, 2, -1)
        save("chk", prefill[0], P0)
        for i in (0, L - 1):
            for part, name in ((0, "k"), (1, "v")):
                with open(os.path.join(root, f"chk__layer.{i}__{name}"), "rb") as f:
                    got = decode_payload(f.read())
                if not np.array_equal(got.reshape(-1), want[i, part]):
                    raise RuntimeError(f"shm file layer {i} {name} differs from the packed frame")
        load("chk", P0)
        back = cache.read_frame("chk", P0, S)
        torch.cuda.synchronize()
        if not torch.equal(back.view(torch.int16), frame.view(torch.int16)):
            raise RuntimeError("shm device load differs from the packed frame")
        if os.listdir(root):
            raise RuntimeError("the load left files behind")
        cache.free("chk")

        reps = max(5, min(args.steps, 20))
        save_ms, load_ms = [], []
        for i in range(max(1, args.warmup) + reps):
            req = f"one{i}"
            torch.cuda.synchronize()
            a = time.perf_counter()
            save(req, prefill[0], S)
            b = time.perf_counter()
            load(req, S)
            c = time.perf_counter()
            cache.free(req)
            if i >= max(1, args.warmup):
                save_ms.append((b - a) * 1e3)
                load_ms.append((c - b) * 1e3)
        sv, ld = statistics.median(save_ms), statistics.median(load_ms)
        tot = statistics.median([x + y for x, y in zip(save_ms, load_ms)])
        batch_ms = []
        for i in range(max(1, args.warmup) + max(3, reps // 2)):
            torch.cuda.synchronize()
            a = time.perf_counter()
            for r, (p, P) in enumerate(zip(prefill, lengths)):
                save(f"b{i}r{r}", p, P)
            for r, P in enumerate(lengths):
                load(f"b{i}r{r}", P)
            t = time.perf_counter() - a
            for r in range(len(lengths)):
                cache.free(f"b{i}r{r}")
            if i >= max(1, args.warmup):
                batch_ms.append(t * 1e3)
        bt = statistics.median(batch_ms)
        handoff = sum(lengths) * TOKEN_BYTES
        out["extra"]["shm_device_path"] = {
            "what": "RngdKVConnector on select_transport('shm'): device save -> /dev/shm -> "
                    "device load into the paged cache (the reference's shm handoff per request)",
            "ms_per_512_request": round(tot, 3), "save_ms": round(sv, 3), "load_ms": round(ld, 3),
            "gbps_512_request": round(S * TOKEN_BYTES / tot / 1e6, 2),
            "batch_ms": round(bt, 3), "batch_gbps": round(handoff / bt / 1e6, 2),
            "batch_lengths": lengths, "reps": reps,
            "files_and_cache_checked": True}
        log(f"shm device path: 512-token request {tot:.2f} ms (save {sv:.2f}, load {ld:.2f}); "
            f"8-request batch {bt:.1f} ms, {handoff / bt / 1e6:.2f} GB/s")
    finally:
        shutil.rmtree(root, ignore_errors=True)
        for k, v in saved_env.items():
            if v is None:
                os.environ.pop(k, None)
            else:
                os.environ[k] = v
        kvt.reset_selection()
        del prefill, cache
        torch.cuda.empty_cache()


def bench_host_link(args, torch, lib, dev, out, dframe):
    """Host-link rates for 64 MiB: DMA-engine copies each way and both at once
    (on two side streams: one engine each way), and a kernel's own stores to /
    loads from pinned memory."""
    from rngd_pd_amd import hip
    from rngd_pd_amd._lib import PDK_COPY_D2H, PDK_COPY_H2D
    nbytes = S * TOKEN_BYTES
    pin_a, pin_b = hip.PinnedBuffer(nbytes), hip.PinnedBuffer(nbytes)
    dbuf = torch.empty(nbytes // 2, dtype=torch.bfloat16, device=dev)
    s1, s2 = torch.cuda.Stream(device=dev), torch.cuda.Stream(device=dev)
    st = s1.cuda_stream

    def check(rc):
        if rc:
            raise RuntimeError(lib.pdk_last_error().decode())

    def d2h(stream=st):
        check(lib.pdk_copy_layers(ctypes.c_void_p(pin_a.ptr), ctypes.c_void_p(dframe.data_ptr()),
                                  nbytes, 1, PDK_COPY_D2H, None, None, stream))

    def h2d(stream=st):
        check(lib.pdk_copy_layers(ctypes.c_void_p(dbuf.data_ptr()), ctypes.c_void_p(pin_b.ptr),
                                  nbytes, 1, PDK_COPY_H2D, None, None, stream))

    def both():
        d2h(st)
        h2d(s2.cuda_stream)

    def kernel_store():
        check(lib.pdk_copy_kernel(ctypes.c_void_p(pin_a.ptr), ctypes.c_void_p(dframe.data_ptr()),
                                  nbytes, st))

    def kernel_load():
        check(lib.pdk_copy_kernel(ctypes.c_void_p(dbuf.data_ptr()), ctypes.c_void_p(pin_b.ptr),
                                  nbytes, st))

    res = {}
    for name, fn, moved in (("dma_d2h_gbps", d2h, nbytes), ("dma_h2d_gbps", h2d, nbytes),
                            ("dma_both_ways_total_gbps", both, 2 * nbytes),
                            ("kernel_store_to_pinned_gbps", kernel_store, nbytes),
                            ("kernel_load_from_pinned_gbps", kernel_load, nbytes)):
        vals = []
        for i in range(6):
            torch.cuda.synchronize()
            a = time.perf_counter()
            fn()
            torch.cuda.synchronize()
            if i:
                vals.append(time.perf_counter() - a)
        res[name] = round(moved / statistics.median(vals) / 1e9, 1)
    out["extra"]["host_link"] = res
    log(f"host link: {res}")
    pin_a.close()
    pin_b.close()


def bench_decode(args, torch, K, lib, dev, out, batches=(4, 8, 16), ctx=512):
    # One paged cache for the largest batch, allocated once as a serving engine
    # reserves its cache at start-up; smaller batches use the first B streams.
    # (Caches re-allocated after memory went back to the driver measured about
    # 9 % slower per layer at B=16.)
    res = {}
    nb_per = (ctx + BS - 1) // BS
    bmax = max(batches)
    nb = bmax * nb_per
    gen = torch.Generator(device=dev).manual_seed(16)
    cache_k = torch.randn((L, nb, H, BS, D), generator=gen, device=dev).to(torch.bfloat16)
    cache_v = torch.randn((L, nb, H, D, BS), generator=gen, device=dev).to(torch.bfloat16)
    q_all = torch.randn((L, bmax, HQ, D), generator=gen, device=dev).to(torch.bfloat16)
    perm = np.random.default_rng(16).permutation(nb).astype(np.int32).reshape(bmax, nb_per)
    tables_all = torch.from_numpy(perm).to(dev)
    out_all = torch.empty((L, bmax, HQ, D), dtype=torch.bfloat16, device=dev)
    for B in batches:
        q = q_all[:, :B]
        outp = out_all[:, :B]
        tables = tables_all[:B]
        ctx_lens = torch.full((B,), ctx, dtype=torch.int32, device=dev)
        wsb = K.workspace_bytes(B, HQ, ctx, D)
        ws = torch.zeros(max(1, wsb // 4), dtype=torch.float32, device=dev)   # split partials
        scale = 1.0 / math.sqrt(D)
        ptrs = [(q[l].data_ptr(), cache_k[l].data_ptr(), cache_v[l].data_ptr(), outp[l].data_ptr())
                for l in range(L)]

        def step(timer=None):
            # Event pairs bracket a whole 32-layer step: per-call pairs around a
            # ~10 us kernel would also time the host's enqueue of the next call.
            st = torch.cuda.current_stream().cuda_stream
            rc = 0
            if timer:
                timer.begin("step")
            for l in range(L):
                qp, kp, vp, op = ptrs[l]
                rc |= lib.pdk_decode_attn(qp, kp, vp, nb, tables.data_ptr(), nb_per,
                                          ctx_lens.data_ptr(), ctx, B, HQ, H, D, scale,
                                          ws.data_ptr(), wsb, op, st)
            if timer:
                timer.end("step")
            if rc:
                raise RuntimeError("decode attention launch failed: " + lib.pdk_last_error().decode())

        for _ in range(args.warmup):
            step()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(args.steps):
            step()
        torch.cuda.synchronize()
        eager = (time.perf_counter() - t0) / args.steps
        # The launches' own time: each step's 32 launches queued behind a 2 ms
        # spin, so the host has enqueued them all before the first starts, and
        # event pairs around the step time the kernels back to back.
        delay = gpu_delay(torch, 2000)
        timer = Timer(torch, args.steps)
        for _ in range(args.steps):
            delay()
            step(timer)
        torch.cuda.synchronize()
        # The same 32-layer step replayed from a HIP graph (no host launch cost).
        g = torch.cuda.CUDAGraph()
        s = torch.cuda.Stream(device=dev)
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            step()
            torch.cuda.synchronize()
            with torch.cuda.graph(g, stream=s):
                step()
        torch.cuda.synchronize()
        graph_ref = outp.clone()
        for _ in range(args.warmup):
            g.replay()
        torch.cuda.synchronize()
        if not torch.equal(outp.view(torch.int16), graph_ref.view(torch.int16)):
            raise RuntimeError("graph replay differs from eager attention")
        # Event pairs around each replay: the graph's own per-launch time.
        gtimer = Timer(torch, args.steps)
        t0 = time.perf_counter()
        for _ in range(args.steps):
            gtimer.begin("graph")
            g.replay()
            gtimer.end("graph")
        torch.cuda.synchronize()
        graphed = (time.perf_counter() - t0) / args.steps
        # The same launches with attention's loads and none of its arithmetic
        # (pdk_attn_read_probe), replayed the same way: the floor of this
        # access pattern, block-id reads included.
        def probe_step():
            for l in range(L):
                K.attn_read_probe(cache_k[l], cache_v[l], tables, ctx_lens, ctx, HQ, outp[l])
        gp = torch.cuda.CUDAGraph()
        with torch.cuda.stream(s):
            probe_step()
            torch.cuda.synchronize()
            with torch.cuda.graph(gp, stream=s):
                probe_step()
        torch.cuda.synchronize()
        for _ in range(args.warmup):
            gp.replay()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(args.steps):
            gp.replay()
        torch.cuda.synchronize()
        probe_us = (time.perf_counter() - t0) / args.steps / L * 1e6
        kv_bytes = B * ctx * H * D * 2 * 2 + 2 * B * HQ * D * 2   # K+V read, q read, out write
        kern = timer.mean_s("step") / L                           # one layer's launch(es)
        kern_graph = gtimer.mean_s("graph") / L
        res[f"B{B}"] = {
            "tokens_per_s_graph": round(B / graphed, 1),
            "tokens_per_s_eager": round(B / eager, 1),
            "step_us_graph": round(graphed * 1e6, 1),
            "step_us_eager": round(eager * 1e6, 1),
            "layer_call_us": round(kern * 1e6, 2),
            "layer_call_us_graph": round(kern_graph * 1e6, 2),
            "layer_us_graph": round(graphed / L * 1e6, 2),
            "read_probe_layer_us_graph": round(probe_us, 2),
            "roofline": roofline(kv_bytes, kern,
                                 measured_traffic("decode_attn_B16") if B == 16 else None),
            "step_hbm_frac_graph": round(L * kv_bytes / graphed / 1e9 / HBM_PEAK_GBS, 4),
        }
        log(f"decode B={B}: graph {graphed*1e6:.1f} us/step ({B/graphed:.0f} tok/s), "
            f"eager {eager*1e6:.1f} us, layer call {kern*1e6:.2f} us "
            f"(graph {kern_graph*1e6:.2f}); "
            f"loads-only probe {probe_us:.2f} us/layer")
        del ws, g, gp
    out["extra"]["decode_batch"] = res
    out["kernels"] = dict(out.get("kernels", {}), decode_attn_B16=res[f"B{batches[-1]}"]["roofline"])


def bench_decode_long(args, torch, K, dev, out, B=16, ctx=2048):
    """Decode attention at a longer context, B=16 x 2048 tokens (134 MB of K+V
    per layer, 4.3 GB for 32 layers): with 128 (stream, KV head) units the
    launch keeps the context in one split (no merge launch; a longer context
    splits it and a merge launch combines the parts). 32 layers replayed from
    a HIP graph, timed with events around the replays."""
    nb_per = ctx // BS
    nb = B * nb_per
    gen = torch.Generator(device=dev).manual_seed(17)
    cache_k = torch.randn((L, nb, H, BS, D), generator=gen, device=dev).to(torch.bfloat16)
    cache_v = torch.randn((L, nb, H, D, BS), generator=gen, device=dev).to(torch.bfloat16)
    q = torch.randn((L, B, HQ, D), generator=gen, device=dev).to(torch.bfloat16)
    tables = torch.from_numpy(np.random.default_rng(17).permutation(nb).astype(np.int32)
                              .reshape(B, nb_per)).to(dev)
    ctx_lens = torch.full((B,), ctx, dtype=torch.int32, device=dev)
    outp = torch.empty_like(q)
    ws = torch.zeros(max(1, K.workspace_bytes(B, HQ, ctx, D) // 4), dtype=torch.float32, device=dev)
    scale = 1.0 / math.sqrt(D)

    def step():
        for l in range(L):
            K.decode_attention(q[l], cache_k[l], cache_v[l], tables, ctx_lens, ctx, scale=scale,
                               out=outp[l], workspace=ws)
    step()
    torch.cuda.synchronize()
    eager_out = outp.clone()
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream(device=dev)
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            step()
    torch.cuda.synchronize()
    for _ in range(max(1, args.warmup)):
        g.replay()
    torch.cuda.synchronize()
    if not torch.equal(outp.view(torch.int16), eager_out.view(torch.int16)):
        raise RuntimeError("graph replay differs from eager attention (ctx 2048)")
    ta, tb = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    reps = max(5, args.steps)
    ta.record()
    for _ in range(reps):
        g.replay()
    tb.record()
    torch.cuda.synchronize()
    us = ta.elapsed_time(tb) * 1e3 / reps / L
    kv_bytes = B * ctx * H * D * 2 * 2 + 2 * B * HQ * D * 2
    out["extra"]["decode_batch_ctx2048"] = {
        f"B{B}": {"layer_us_graph": round(us, 2),
                  "tokens_per_s_graph": round(B / (us * L) * 1e6, 1),
                  "roofline": roofline(kv_bytes, us * 1e-6)}}
    log(f"decode B={B} ctx={ctx}: {us:.2f} us per layer (graph, attention and any merge), "
        f"{kv_bytes / us / 1e3:.0f} GB/s")
    del g, cache_k, cache_v
    torch.cuda.empty_cache()


def bench_attn_floor(args, torch, K, dev, out, batches=(4, 8, 16), ctx=512):
    """What one launch per layer can reach at decode attention's sizes: 32
    launches of the one-shot read probe (one 16-byte vector per lane, a
    workgroup per 4 KiB) over the bytes of one layer's K and V (B x ctx x 8
    heads x 128 dims x 2 x 2 B), each layer its own buffer (1.07 GB in all at
    B=16, so nothing comes from the 256 MB last-level cache), replayed from a
    HIP graph as the attention leg is; and 32 launches of a one-workgroup probe,
    the graph's per-kernel cadence. Attention also loads its block tables
    before it can address K and V, a dependent round trip the probe does not
    pay."""
    res = {}
    for B in batches:
        nbytes = B * ctx * H * D * 2 * 2
        bufs = [torch.empty(nbytes, dtype=torch.uint8, device=dev).fill_(1) for _ in range(L)]
        row = {}
        for label, size in (("read_once", nbytes), ("empty", 4096)):
            def step():
                for l in range(L):
                    K.stream_probe("read", src=bufs[l], nbytes=size)
            step()
            torch.cuda.synchronize()
            g = torch.cuda.CUDAGraph()
            s = torch.cuda.Stream(device=dev)
            s.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(s):
                with torch.cuda.graph(g, stream=s):
                    step()
            torch.cuda.synchronize()
            for _ in range(3):
                g.replay()
            ta, tb = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            reps = max(5, args.steps)
            ta.record()
            for _ in range(reps):
                g.replay()
            tb.record()
            torch.cuda.synchronize()
            us = ta.elapsed_time(tb) * 1e3 / reps / L
            row[label] = {"us_per_layer": round(us, 2)}
            if size == nbytes:
                row[label]["frac"] = round(nbytes / us / 1e3 / HBM_PEAK_GBS, 4)
            del g
        res[f"B{B}"] = row
        del bufs
        torch.cuda.empty_cache()
    out["extra"]["decode_attn_read_floor"] = res
    log("attention read floor (us per layer, one-shot read / empty launch): " + ", ".join(
        f"B={B} {res[f'B{B}']['read_once']['us_per_layer']} / {res[f'B{B}']['empty']['us_per_layer']}"
        for B in batches))


def bench_step(args, torch, dev, out, batches=(4, 16), ctx=512):
    """Full Llama-3.1-8B decode step (32 layers, random-init bf16 weights, no
    checkpoint): embed + the rows' sums of squares -> per layer q|k|v GEMM
    split over K (rows scaled by the pre-attention RMSNorm's factor), RoPE +
    new-token cache write + paged decode attention in one kernel, o GEMM +
    residual (+ its sums of squares), gate|up GEMM with the post-attention
    norm's row scale and SwiGLU, down GEMM split over K whose last split adds
    the residual (+ sums of squares) -> lm_head GEMM with the final norm's row
    scale and the greedy argmax. The norms' gains are folded into the
    decoder's tiled copies of the weights, which the GEMMs read. Every
    stream at context ctx (its new token at slot ctx-1; the reference's S=512
    step attends over the whole S). Bytes per step = every weight read once
    (16.06 GB; the embedding contributes B rows) + the K/V of all layers."""
    from rngd_pd_amd.engines.llama_decode import LlamaConfig, LlamaDecoder, LlamaWeights
    from rngd_pd_amd.engines.paged_cache import PagedKVCache
    published = {4: 21.54, 16: 35.54}           # ms/step, bench/profile_solo_S512_B{4,16}.json
    cfg = LlamaConfig()
    t0 = time.perf_counter()
    w = LlamaWeights.random(cfg, seed=8, device=dev)
    bmax = max(batches)
    per = (ctx + BS - 1) // BS
    cache = PagedKVCache(cfg.n_layers, bmax * per, H, D, device=dev)
    gen = torch.Generator(device=dev).manual_seed(9)
    for li in range(cfg.n_layers):
        cache.k[li].copy_(torch.randn(cache.k[li].shape, generator=gen, device=dev))
        cache.v[li].copy_(torch.randn(cache.v[li].shape, generator=gen, device=dev))
    dec = LlamaDecoder(w, cache, max_batch=bmax)
    perm = np.random.default_rng(9).permutation(bmax * per).astype(np.int32).reshape(bmax, per)
    tables_all = torch.from_numpy(perm).to(dev)
    torch.cuda.synchronize()
    log(f"step: weights {w.nbytes() / 1e9:.2f} GB ready in {time.perf_counter() - t0:.1f} s")
    weight_bytes = w.nbytes() - w.embed.numel() * 2
    res = {}
    for B in batches:
        tables = tables_all[:B].contiguous()
        ctx_d = torch.full((B,), ctx, dtype=torch.int32, device=dev)
        tok = torch.randint(0, cfg.vocab, (B,), generator=gen, device=dev)
        for _ in range(args.warmup):
            dec.step(tok, ctx_d, tables, ctx)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(args.steps):
            dec.step(tok, ctx_d, tables, ctx)
        torch.cuda.synchronize()
        eager = (time.perf_counter() - t0) / args.steps
        want = dec.tokens[:B].clone()
        g = dec.capture(tok, ctx_d, tables, ctx)
        for _ in range(args.warmup):
            g.replay()
        torch.cuda.synchronize()
        if not torch.equal(dec.tokens[:B], want):
            raise RuntimeError("graph replay of the decode step differs from the eager step")
        ta, tb = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0 = time.perf_counter()
        ta.record()
        for _ in range(args.steps):
            g.replay()
        tb.record()
        torch.cuda.synchronize()
        graphed = (time.perf_counter() - t0) / args.steps
        dev_ms = ta.elapsed_time(tb) / args.steps
        step_bytes = weight_bytes + B * H * 2 + cfg.n_layers * B * ctx * H * D * 2 * 2
        ms = graphed * 1e3
        res[f"B{B}"] = {
            "ms_per_step_graph": round(ms, 3),
            "ms_per_step_eager": round(eager * 1e3, 3),
            "tokens_per_s_graph": round(B / graphed, 1),
            "bytes_per_step": step_bytes,
            "hbm_gbps": round(step_bytes / (dev_ms / 1e3) / 1e9, 1),
            "hbm_frac": round(step_bytes / (dev_ms / 1e3) / 1e9 / HBM_PEAK_GBS, 4),
            "reference_ms_per_step": published[B],
            "speedup_vs_reference": round(published[B] / ms, 2),
            "weight_layout": "tiled" if dec.tiled else "out_in",
        }
        log(f"step B={B} ctx={ctx}: graph {ms:.3f} ms ({B / graphed:.0f} tok/s, "
            f"{res[f'B{B}']['hbm_frac'] * 100:.1f}% of HBM), eager {eager * 1e3:.3f} ms; "
            f"reference {published[B]} ms")
        del g
    out["extra"]["decode_step_llama8b"] = res
    del dec, cache, w
    torch.cuda.empty_cache()


def bench_serve(args, out):
    """Two prefill producer processes and one decode consumer on this
    GPU (same-GPU IPC handoff, continuous batching at width 16), 64 requests
    with Poisson(20/s) arrivals, prompts U[128,1024], 128 greedy tokens each,
    random-init Llama-3.1-8B weights. Runs rngd_pd_amd.serving.pd_one_gpu as a
    child process and records its summary: three passes of the same seeded
    workload on the same processes (the first pass's figures at the top level,
    every pass under "passes", the spread under "across_passes"), each with its
    decode steps grouped by how many prefills overlapped them and its time to
    first token split into queueing and prefill."""
    import subprocess
    cmd = [sys.executable, "-u", "-m", "rngd_pd_amd.serving.pd_one_gpu", "run",
           "--requests", "64", "--rate", "20", "--min-len", "128", "--max-len", "1024",
           "--max-new", "128", "--batch", "16", "--producers", "2", "--seed", "0",
           "--repeats", "3"]
    log("serve: " + " ".join(cmd[3:]))
    r = subprocess.run(cmd, stdout=subprocess.PIPE, text=True, timeout=900,
                       cwd=os.path.dirname(os.path.abspath(__file__)))
    if r.returncode != 0:
        raise RuntimeError(f"pd_one_gpu exited with {r.returncode}")
    summary = json.loads([ln for ln in r.stdout.splitlines() if ln.startswith("{")][-1])
    out["extra"]["pd_one_gpu"] = summary
    for i, p in enumerate(summary.get("passes", [summary])):
        log(f"serve pass {i}: {p['output_tokens_per_s']} tok/s, TTFT p50 {p['ttft_ms']['p50']} ms "
            f"(queued {p['ttft_parts_ms']['queued_p50']}, prefill {p['ttft_parts_ms']['prefill_p50']}), "
            f"TPOT p50/p90 {p['tpot_ms']['p50']}/{p['tpot_ms']['p90']} ms, steps by overlapping "
            f"prefills {p['decode_steps_by_overlapping_prefills']}")


def bench_long(args, torch, dev, out, n_req=16, T=2048, hidden=4096):
    """Long-context layer-pipelined save: n_req requests of T tokens (Llama-3.1-8B
    KV), 32 layers. Per layer the "prefill" runs a bf16 GEMM [n_req*T, hidden] x
    [hidden, hidden] on the compute stream, then save_kv_layer for every request
    (the connector's device path: side-stream pack -> pinned D2H -> one ordered
    writer thread per request publishing byte-identical wire files into /dev/shm).
    Times the GEMMs alone, the saves alone and both; overlap % = hidden share of
    the shorter leg. T = 2048 tokens per request is this workload's choice (the
    prefill GEMM's row count is not fixed by the reference)."""
    import shutil
    from rngd_pd_amd.connector.rngd_kv import KVConnectorRole, RngdKVConnector
    from rngd_pd_amd.connector.transport import ShmTransport
    gen = torch.Generator(device=dev).manual_seed(4)
    kv = [torch.randn((L, 2, T, H, D), generator=gen, device=dev).to(torch.bfloat16)
          for _ in range(n_req)]
    x = torch.randn((n_req * T, hidden), generator=gen, device=dev).to(torch.bfloat16)
    w = torch.randn((hidden, hidden), generator=gen, device=dev).to(torch.bfloat16)
    y = torch.empty((n_req * T, hidden), dtype=torch.bfloat16, device=dev)
    wire_bytes = n_req * L * 2 * H * D * T * 2

    def run(gemm, save, tag):
        root = tempfile.mkdtemp(prefix="rngd_long_", dir="/dev/shm" if os.path.isdir("/dev/shm")
                                else None)
        conns = [RngdKVConnector(KVConnectorRole.WORKER, req_id=f"{tag}{i}",
                                 transport=ShmTransport(root), n_layers=L, frame_tokens=T)
                 for i in range(n_req)] if save else []
        try:
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            for l in range(L):
                if gemm:
                    torch.matmul(x, w, out=y)
                for i, c in enumerate(conns):
                    c.save_kv_layer(f"layer.{l}", (kv[i][l, 0], kv[i][l, 1]), num_tokens=T)
            for c in conns:
                c.wait_for_save()
            torch.cuda.synchronize()
            dt = time.perf_counter() - t0
            if save:
                n_files = len(os.listdir(root))
                if n_files != n_req * L * 2:
                    raise RuntimeError(f"long-context save published {n_files} files, "
                                       f"expected {n_req * L * 2}")
            return dt
        finally:
            for c in conns:
                c.close()
            shutil.rmtree(root, ignore_errors=True)

    run(True, True, "warm")                         # allocations, envelopes, clocks
    reps = {"g": [], "s": [], "b": []}
    for rep in range(3):                            # interleaved; the save leg is host-bound
        reps["g"].append(run(True, False, f"g{rep}-"))
        reps["s"].append(run(False, True, f"s{rep}-"))
        reps["b"].append(run(True, True, f"b{rep}-"))
    t_gemm, t_save, t_both = (statistics.median(reps[k]) for k in ("g", "s", "b"))
    overlap = (t_gemm + t_save - t_both) / min(t_gemm, t_save)
    flops = 2.0 * n_req * T * hidden * hidden * L
    res = {"repeats": 3, "requests": n_req, "tokens_per_request": T, "gemm": f"[{n_req * T},{hidden}]x[{hidden},{hidden}] bf16 per layer",
           "wire_bytes": wire_bytes, "ms_gemm_only": round(t_gemm * 1e3, 2),
           "ms_save_only": round(t_save * 1e3, 2), "ms_both": round(t_both * 1e3, 2),
           "overlap_pct": round(100 * max(0.0, min(1.0, overlap)), 1),
           "save_gbps": round(wire_bytes / t_save / 1e9, 2),
           "save_gbps_with_gemm": round(wire_bytes / t_both / 1e9, 2),
           "gemm_tflops": round(flops / t_gemm / 1e12, 1)}
    out["extra"]["long_context"] = res
    log(f"long context: gemm {res['ms_gemm_only']} ms, save {res['ms_save_only']} ms, "
        f"both {res['ms_both']} ms, overlap {res['overlap_pct']} %, save {res['save_gbps']} GB/s")
    del kv, x, w, y


def bench_cpu(args, out):
    """The reference CPU shm path (oracle restatement), bounded to ~cpu_seconds."""
    from oracle import wire
    lengths = out["config"].get("lengths") or workload()
    root_parent = "/dev/shm" if os.access("/dev/shm", os.W_OK) else None
    root = tempfile.mkdtemp(prefix="pdk_cpu_baseline.", dir=root_parent)
    times, moved, reqs = [], 0, 0
    try:
        data = []
        budget_t0 = time.perf_counter()
        for i, P in enumerate(lengths):
            Kf = wire.make_kv(100 + i, (L, H, D, S))
            Vf = wire.make_kv(200 + i, (L, H, S, D))
            Kf[:, :, :, P:] = 0.0
            Vf[:, :, P:, :] = 0.0
            data.append((P, Kf, Vf))
            if time.perf_counter() - budget_t0 > args.cpu_seconds / 2:
                break
        wire.cpu_shm_handoff(root, "warm", data[0][1], data[0][2])
        t_start = time.perf_counter()
        while True:
            for i, (P, Kf, Vf) in enumerate(data):
                Kg, Vg, sec = wire.cpu_shm_handoff(root, f"r{reqs}", Kf, Vf)
                if not (np.array_equal(Kg.view(np.uint32), Kf.view(np.uint32))
                        and np.array_equal(Vg.view(np.uint32), Vf.view(np.uint32))):
                    raise RuntimeError("CPU shm round trip is not byte-exact")
                times.append(sec)
                moved += P * TOKEN_BYTES
                reqs += 1
            if time.perf_counter() - t_start > args.cpu_seconds:
                break
        wall = sum(times)
    finally:
        for f in os.listdir(root):
            os.unlink(os.path.join(root, f))
        os.rmdir(root)
    cores_avail = len(os.sched_getaffinity(0))
    out["cpu_baseline"] = {
        "value": round(moved / wall / 1e9, 3), "unit": "GB/s", "cores": 1, "kind": "port",
        "sample": (f"{reqs} requests ({len(data)} distinct of the batch's lengths, S=512 frames, "
                   f"64 MiB bf16 each on the wire) through ser -> /dev/shm tmp+fsync+rename -> "
                   f"read -> deser -> f32 place, single thread, {wall:.1f} s; "
                   f"{cores_avail} cores visible"),
        "ms_per_request_median": round(statistics.median(times) * 1e3, 2),
    }
    log(f"cpu baseline: {out['cpu_baseline']['value']} GB/s, "
        f"{out['cpu_baseline']['ms_per_request_median']} ms/request")
    bench_cpu_attention(args, out)


def bench_cpu_attention(args, out, B=16, ctx=512):
    """Decode attention's CPU baseline: the oracle's fp32 restatement of
    cpu_layer's attention (numpy einsum, one thread), on a bounded sample of
    the B=16, context 512 layers the GPU leg runs."""
    from oracle import attention as oatt
    rng = np.random.default_rng(3)
    NKV, HQ_, HD = H, HQ, D
    q = rng.standard_normal((B, HQ_, HD)).astype(np.float32)
    Kd = rng.standard_normal((B, NKV, HD, ctx)).astype(np.float32)
    Vd = rng.standard_normal((B, NKV, ctx, HD)).astype(np.float32)
    pos = [ctx - 1] * B
    oatt.cpu_attention(q, Kd, Vd, pos)                         # warm
    times = []
    t0 = time.perf_counter()
    while not times or (time.perf_counter() - t0 < min(5.0, args.cpu_seconds / 2)
                        and len(times) < 64):
        t = time.perf_counter()
        oatt.cpu_attention(q, Kd, Vd, pos)
        times.append(time.perf_counter() - t)
    per_layer = statistics.median(times)
    out["extra"]["cpu_baseline_attention"] = {
        "tokens_per_s": round(B / (per_layer * L), 2), "unit": "tokens/s (attention-only step)",
        "ms_per_layer": round(per_layer * 1e3, 3), "threads": 1, "kind": "port",
        "sample": f"{len(times)} layers of B={B}, context {ctx}, Hq {HQ_}, Hkv {NKV}, fp32 numpy "
                  f"einsum (no BLAS), median per layer x {L} layers per step"}
    log(f"cpu attention baseline: {per_layer * 1e3:.2f} ms/layer, "
        f"{out['extra']['cpu_baseline_attention']['tokens_per_s']} tokens/s")


def bench_copy(args, torch, K, dev, out):
    """Streaming ceilings and counter calibration.

    First the plain copy kernel over --copy-mib MiB (the known byte count the
    FETCH_SIZE / WRITE_SIZE counters are scaled against). Then the streaming
    probes -- a linear read, a linear write and a copy -- over 256 MiB, 1 GiB
    and 4 GiB, with ordinary and non-temporal accesses, one-shot (one 16-byte
    vector per lane, a workgroup per 4 KiB) and as a grid-stride loop of 8192
    workgroups with four vectors in flight per lane, each timed with HIP events
    on its launch stream (median of --steps launches). The 4 GiB rows are the HBM
    ceilings: 16x the 256 MB last-level cache, so nothing is served from it;
    the smaller rows show how much that cache lifts a repeated stream."""
    n = args.copy_mib << 20
    a = torch.empty(n, dtype=torch.uint8, device=dev).fill_(1)
    b = torch.empty_like(a)
    for _ in range(args.warmup + args.steps):
        K.copy_kernel(b, a)
    torch.cuda.synchronize()
    del a, b
    big = 4 << 30
    src = torch.empty(big, dtype=torch.uint8, device=dev).fill_(3)
    dst = torch.empty(big, dtype=torch.uint8, device=dev)
    rows = []
    for size in (256 << 20, 1 << 30, big):
        for kind in ("read", "write", "copy"):
            for nt in (False, True):
                for blocks in (0, 8192):
                    nbytes = size // 2 if kind == "copy" else size   # a copy moves size in total
                    kw = dict(src=src if kind != "write" else None,
                              dst=dst if kind != "read" else None,
                              nbytes=nbytes, nontemporal=nt, blocks=blocks)
                    timer = Timer(torch, 4 * args.steps)
                    for i in range(args.warmup + args.steps):
                        if i >= args.warmup:
                            timer.begin("p")
                        K.stream_probe(kind, **kw)
                        if i >= args.warmup:
                            timer.end("p")
                    torch.cuda.synchronize()
                    sec = timer.median_s("p")
                    rows.append({"kind": kind, "mib": size >> 20, "nontemporal": nt,
                                 "blocks": blocks, "us": round(sec * 1e6, 2),
                                 "gbps": round(size / sec / 1e9, 1)})
    best = {}
    for r in rows:
        if r["mib"] == big >> 20 and r["gbps"] > best.get(r["kind"], {}).get("gbps", 0):
            best[r["kind"]] = dict(r, frac=round(r["gbps"] / HBM_PEAK_GBS, 4))
    out["extra"]["streaming_ceilings"] = {"hbm_4gib": best, "sweep": rows}
    log("streaming ceilings (4 GiB, best of ordinary / non-temporal, one-shot / grid-stride): "
        + ", ".join(f"{k} {v['gbps']} GB/s ({v['frac'] * 100:.1f}%)" for k, v in best.items()))
    for r in rows:
        shape = "one-shot" if r["blocks"] == 0 else f"wg={r['blocks']}"
        log(f"  {r['kind']:5s} {r['mib']:5d} MiB nt={int(r['nontemporal'])} {shape:9s}: "
            f"{r['us']:9.1f} us {r['gbps']:7.1f} GB/s")
    del src, dst
    torch.cuda.empty_cache()


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this package has no multi-GPU path "
              f"(--gpus {args.gpus} requested). Run with --gpus 1.", file=sys.stderr)
        return 2
    import torch
    from rngd_pd_amd import kernels as K
    from rngd_pd_amd import _lib
    lib = _lib.lib()
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        return 1
    dev = torch.device("cuda:0")
    # No cyclic collection inside timed loops: a full collection is a host
    # stall of tens of milliseconds that the GPU sees as idle time.
    gc.collect()
    gc.disable()
    out = {"metric": METRIC, "value": None, "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
           "warmup": args.warmup, "ms_per_step": None, "higher_is_better": True,
           "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
           "data": "synthetic: seeded N(0,1) bf16 KV; request lengths U[64,512] from seed 0",
           "config": {"workload": "KV handoff batch: 8 Llama-3.1-8B requests, lengths U[64,512], "
                                  "pack -> DMA of the valid columns into pinned host S=512 wire "
                                  "frames (zero tails by host threads) -> DMA back up -> scatter "
                                  "into a paged cache (block 16, permuted block table), "
                                  "pipelined across requests and layers",
                      "layers": L, "kv_heads": H, "head_dim": D, "frame_tokens": S,
                      "block_size": BS},
           "extra": {}}
    if args.legs == {"copy"}:
        bench_copy(args, torch, K, dev, out)
        print(json.dumps(out), flush=True)
        return 0
    if args.legs & {"all", "handoff"}:
        bench_handoff(args, torch, K, lib, dev, out)
    if args.legs & {"all", "shm"}:
        bench_shm(args, torch, K, dev, out)
    if args.legs & {"all", "decode"}:
        bench_decode(args, torch, K, lib, dev, out)
        bench_decode_long(args, torch, K, dev, out)
        bench_attn_floor(args, torch, K, dev, out)
    if args.legs & {"all", "step"}:
        bench_step(args, torch, dev, out)
    if args.legs & {"all", "long"}:
        bench_long(args, torch, dev, out)
    if args.legs & {"all", "serve"}:
        bench_serve(args, out)
    if "all" in args.legs and args.cpu_seconds > 0:
        bench_cpu(args, out)
    if args.legs == {"step"}:
        b = out["extra"]["decode_step_llama8b"]["B16"]
        out.update(value=b["tokens_per_s_graph"], unit="tokens/s",
                   ms_per_step=b["ms_per_step_graph"])
    if args.legs == {"decode"}:
        b = out["extra"]["decode_batch"]["B16"]
        out.update(value=b["tokens_per_s_graph"], unit="tokens/s",
                   ms_per_step=b["step_us_graph"] / 1e3, roofline=b["roofline"])
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
