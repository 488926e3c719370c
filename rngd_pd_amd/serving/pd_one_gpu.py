"""Prefill/decode disaggregation on one GPU: N prefill producers, one decode consumer.

The reference runs prefill and decode as separate workers behind a gateway
(serving/cluster.py: PrefillWorker, DecodeWorkerBase, _ContinuousScheduler)
and hands KV over /dev/shm. Here all of them share one MI355X:

  orchestrator (no GPU)  seeded Poisson arrivals, prompts routed round-robin
       |  JSON lines over pipes
  producer x N           LlamaPrefill -> RngdKVConnector.save_kv_layer per layer
       |                 on the ipc transport (frames stay in the producer's HBM)
  consumer               ContinuousScheduler: loader threads scatter each frame
                         from the producer's memory into the paged cache; the
                         decode step (LlamaDecoder, HIP graphs) runs the batch

Every process builds the same random-init weights from one seed (no
checkpoint). The orchestrator reports time to first token (arrival to the
producer's first token), per-request end-to-end latency, decode TPOT and the
output-token throughput of the run.

  python -m rngd_pd_amd.serving.pd_one_gpu run [--requests 64 --rate 20 ...]
  python -m rngd_pd_amd.serving.pd_one_gpu control ...   (one process, B=1, for tests)
"""
import argparse
import json
import math
import os
import queue
import shutil
import subprocess
import sys
import tempfile
import threading
import time

_LOCK = threading.Lock()


def _say(obj):
    with _LOCK:
        sys.stdout.write(json.dumps(obj) + "\n")
        sys.stdout.flush()


def _log(msg):
    print(f"[pd] {msg}", file=sys.stderr, flush=True)


def model_config(args):
    from ..engines.llama_decode import LlamaConfig
    if args.small:
        return LlamaConfig(hidden=512, n_heads=8, n_kv_heads=2, head_dim=128, inter=1024,
                           vocab=1000, n_layers=args.layers or 2)
    return LlamaConfig(n_layers=args.layers or 32)


def frame_tokens(args):
    return (args.max_len + 15) // 16 * 16


def workload(args, rep=0):
    """Seeded arrivals (exponential gaps at ``rate``/s), prompt lengths
    U[min_len, max_len] and prompt token ids U[0, vocab). Every pass of a run
    replays the same workload under request ids of its own."""
    import numpy as np
    rng = np.random.default_rng(args.seed)
    vocab = model_config(args).vocab
    t, out = 0.0, []
    prefix = "q" if rep == 0 else f"r{rep}q"
    for i in range(args.requests):
        t += float(rng.exponential(1.0 / args.rate))
        n = int(rng.integers(args.min_len, args.max_len + 1))
        out.append({"req": f"{prefix}{i}", "arrival": t,
                    "tokens": rng.integers(0, vocab, n).tolist()})
    return out


# ---------------------------------------------------------------------------
# producer
# ---------------------------------------------------------------------------
def producer(args):
    import torch
    from ..connector.ipc import IpcTransport
    from ..connector.rngd_kv import KVConnectorRole, RngdKVConnector
    from ..engines.llama_decode import LlamaWeights
    from ..engines.llama_prefill import LlamaPrefill
    cfg = model_config(args)
    w = LlamaWeights.random(cfg, seed=args.seed, device="cuda")
    pre = LlamaPrefill(w, max_tokens=frame_tokens(args))
    t = IpcTransport(args.root, n_slots=args.ipc_slots)
    S = frame_tokens(args)
    # Warm the library paths at prompt lengths across the served range: the
    # GEMM library picks (and loads on first use) a kernel per shape, which
    # otherwise lands on the first requests' time to first token.
    for n in sorted({16, args.min_len, args.max_len, *range(args.min_len, args.max_len, 128)}):
        pre.forward([1] * max(1, min(n, S)))
    torch.cuda.synchronize()
    _say({"ev": "ready", "role": "producer", "pid": os.getpid()})
    for line in sys.stdin:
        msg = json.loads(line)
        if msg.get("cmd") == "stop":
            break
        req, tokens = msg["req"], msg["tokens"]
        t0 = time.monotonic()
        conn = RngdKVConnector(KVConnectorRole.WORKER, req_id=req, transport=t,
                               n_layers=cfg.n_layers, frame_tokens=S)
        T = len(tokens)
        first, _k, _v = pre.forward(
            tokens, on_layer=lambda li, k, v: conn.save_kv_layer(f"layer.{li}", (k, v),
                                                                 num_tokens=T))
        conn.wait_for_save()
        conn.close()
        _say({"ev": "prefilled", "req": req, "first": first, "P": T, "t0": t0,
              "t": time.monotonic(), "prefill_ms": round((time.monotonic() - t0) * 1e3, 2)})
    t.close()
    _say({"ev": "exit", "role": "producer"})


# ---------------------------------------------------------------------------
# consumer
# ---------------------------------------------------------------------------
def consumer(args):
    import torch
    from ..connector.ipc import IpcTransport, close_opened
    from ..connector.rngd_kv import KVConnectorRole, RngdKVConnector
    from ..engines.llama_decode import LlamaDecoder, LlamaWeights
    from ..engines.paged_cache import PagedKVCache
    from .scheduler import ContinuousScheduler
    cfg = model_config(args)
    w = LlamaWeights.random(cfg, seed=args.seed, device="cuda")
    per = math.ceil((args.max_len + args.max_new) / 16)
    cache = PagedKVCache(cfg.n_layers, per * (args.requests + args.batch), cfg.n_kv_heads,
                         cfg.head_dim, device="cuda")
    dec = LlamaDecoder(w, cache, max_batch=args.batch,
                       plan_batch=max(args.batch, args.plan_batch))
    t = IpcTransport(args.root)
    S = frame_tokens(args)

    def produce(item):
        t0 = time.monotonic()
        view = cache.view(item["req_id"], item["P"], S)
        conn = RngdKVConnector(KVConnectorRole.WORKER, req_id=item["req_id"], transport=t,
                               n_layers=cfg.n_layers)
        conn.register_kv_caches(view)
        conn.start_load_kv()
        for i in range(cfg.n_layers):
            conn.wait_for_layer_load(f"layer.{i}")
        conn.close()
        return item["first"], item["P"], (time.monotonic() - t0) * 1e3

    sched = ContinuousScheduler(args.batch, dec, cache, produce, max_blocks=per,
                                use_graphs=not args.eager)
    sched.warmup()
    _say({"ev": "ready", "role": "consumer", "pid": os.getpid()})

    def watch(item):
        item["ev"].wait()
        if item["err"] is not None:
            _say({"ev": "failed", "req": item["req_id"], "error": repr(item["err"])})
        else:
            _say({"ev": "done", "req": item["req_id"], "t": time.monotonic(), **item["out"]})

    watchers = []
    for line in sys.stdin:
        msg = json.loads(line)
        if msg.get("cmd") == "stop":
            break
        if msg.get("cmd") == "steplog":
            _say({"ev": "steplog", "steps": [[round(t, 6), round(d, 3), b]
                                             for t, d, b in sched.take_step_log()]})
            continue
        item = sched.submit_async({"req_id": msg["req"], "first": msg["first"], "P": msg["P"],
                                   "max_new": msg["max_new"]})
        th = threading.Thread(target=watch, args=(item,), daemon=True)
        th.start()
        watchers.append(th)
    for th in watchers:
        th.join()
    sched.close()
    torch.cuda.synchronize()
    close_opened()
    _say({"ev": "exit", "role": "consumer", "steps": sched.steps,
          "occupancy": round(sched.lane_steps / max(sched.steps, 1), 2)})


# ---------------------------------------------------------------------------
# one-process control (B = 1, no handoff between processes)
# ---------------------------------------------------------------------------
def control(args):
    """Prefill and decode each request in one process, one at a time: the
    tokens a correct disaggregated run must reproduce at any --batch (the
    decoder plans its attention for the consumer's plan batch)."""
    import torch
    from ..engines.llama_decode import LlamaDecoder, LlamaWeights
    from ..engines.llama_prefill import LlamaPrefill
    from ..engines.paged_cache import PagedKVCache
    from ..kernels import handoff as K
    cfg = model_config(args)
    w = LlamaWeights.random(cfg, seed=args.seed, device="cuda")
    pre = LlamaPrefill(w, max_tokens=frame_tokens(args))
    per = math.ceil((args.max_len + args.max_new) / 16)
    cache = PagedKVCache(cfg.n_layers, per + 1, cfg.n_kv_heads, cfg.head_dim, device="cuda")
    # The consumer's attention plan (plan_batch), so that a correct run
    # reproduces these tokens exactly whatever batches it forms.
    dec = LlamaDecoder(w, cache, max_batch=1, plan_batch=max(args.batch, args.plan_batch))
    S = frame_tokens(args)
    for r in workload(args):
        first, k, v = pre.forward(r["tokens"])
        P = len(r["tokens"])
        cache.allocate(r["req"], P)
        frame = K.pack_kv(k, v, P, S)
        K.scatter_paged(frame, cache.table(r["req"]), P, S, cache.k, cache.v)
        outs, cur = [first], first
        for pos in range(P, P + args.max_new - 1):
            cache.ensure(r["req"], pos + 1)
            blocks = cache.blocks(r["req"]) + [-1] * (per - len(cache.blocks(r["req"])))
            tab = torch.tensor([blocks], dtype=torch.int32, device="cuda")
            tok = dec.step(torch.tensor([cur], device="cuda"),
                           torch.tensor([pos + 1], dtype=torch.int32, device="cuda"), tab,
                           per * 16)
            cur = int(tok[0].item())
            outs.append(cur)
        cache.free(r["req"])
        _say({"ev": "done", "req": r["req"], "tokens": outs, "P": P})


# ---------------------------------------------------------------------------
# orchestrator
# ---------------------------------------------------------------------------
def _child(role, args, root, env):
    cmd = [sys.executable, "-u", "-m", "rngd_pd_amd.serving.pd_one_gpu", role, "--root", root,
           "--seed", str(args.seed), "--requests", str(args.requests),
           "--min-len", str(args.min_len), "--max-len", str(args.max_len),
           "--max-new", str(args.max_new), "--batch", str(args.batch),
           "--ipc-slots", str(args.ipc_slots), "--layers", str(args.layers or 0),
           "--plan-batch", str(args.plan_batch)]
    if args.small:
        cmd.append("--small")
    if args.eager:
        cmd.append("--eager")
    return subprocess.Popen(cmd, stdin=subprocess.PIPE, stdout=subprocess.PIPE, env=env,
                            text=True, bufsize=1)


def _pump(name, proc, events):
    for line in proc.stdout:
        line = line.strip()
        if line.startswith("{"):
            events.put((name, json.loads(line)))
    events.put((name, {"ev": "eof"}))


def _pct(xs, q):
    xs = sorted(xs)
    return xs[min(len(xs) - 1, int(q * len(xs)))] if xs else None


def contention(steps, prefills, t0, t_end):
    """What the decode steps of one pass shared the GPU with.

    steps: [(start s, ms, streams)] from the consumer; prefills: [(start s,
    end s)] from the producers (one clock: CLOCK_MONOTONIC, system-wide).
    Steps are grouped by how many prefills overlapped them; for each group the
    count and the step-time p50 / p90 (the decode step is one HIP-graph replay,
    so its time is the GPU's answer to what else was running)."""
    out = {}
    for t, ms, b in steps:
        if not t0 <= t <= t_end:
            continue
        e = t + ms / 1e3
        k = sum(1 for a, z in prefills if a < e and z > t)
        out.setdefault(k, []).append(ms)
    return {f"{k}_prefills": {"steps": len(v), "step_ms_p50": round(_pct(v, 0.5), 3),
                              "step_ms_p90": round(_pct(v, 0.9), 3)}
            for k, v in sorted(out.items())}


def _pass(args, rep, procs, names, events):
    """Feed one pass of the workload at its arrival times and collect it."""
    work = workload(args, rep)
    results, firsts, failed = {}, {}, []
    t0 = time.monotonic()
    arrivals = {r["req"]: t0 + r["arrival"] for r in work}
    nxt = 0
    while len(results) + len(failed) < len(work):
        now = time.monotonic()
        while nxt < len(work) and arrivals[work[nxt]["req"]] <= now:
            r = work[nxt]
            p = procs[names[1 + nxt % args.producers]]
            p.stdin.write(json.dumps({"cmd": "prefill", "req": r["req"],
                                      "tokens": r["tokens"]}) + "\n")
            p.stdin.flush()
            nxt += 1
        wait = (arrivals[work[nxt]["req"]] - time.monotonic()) if nxt < len(work) else 1.0
        try:
            n, ev = events.get(timeout=max(0.0005, min(wait, 1.0)))
        except queue.Empty:
            continue
        if ev["ev"] == "prefilled":
            firsts[ev["req"]] = ev
            procs["consumer"].stdin.write(json.dumps({
                "cmd": "decode", "req": ev["req"], "first": ev["first"], "P": ev["P"],
                "max_new": args.max_new}) + "\n")
            procs["consumer"].stdin.flush()
        elif ev["ev"] == "done":
            results[ev["req"]] = ev
        elif ev["ev"] == "failed":
            failed.append(ev)
            _log(f"failed: {ev}")
        elif ev["ev"] == "eof":
            raise RuntimeError(f"{n} exited during the run")
    t_end = time.monotonic()
    procs["consumer"].stdin.write(json.dumps({"cmd": "steplog"}) + "\n")
    procs["consumer"].stdin.flush()
    while True:
        n, ev = events.get(timeout=args.timeout)
        if ev["ev"] == "steplog":
            steps = ev["steps"]
            break
        if ev["ev"] == "eof":
            raise RuntimeError(f"{n} exited during the run")
    ttft = [(firsts[r]["t"] - arrivals[r]) * 1e3 for r in results]
    queued = [(firsts[r]["t0"] - arrivals[r]) * 1e3 for r in results]
    e2e = [(results[r]["t"] - arrivals[r]) * 1e3 for r in results]
    tpot = [results[r]["tpot_ms"] for r in results]
    step_ms = [ms for t, ms, b in steps if t0 <= t <= t_end]
    n_tok = sum(len(results[r]["tokens"]) for r in results)
    summary = {
        "requests": len(work), "completed": len(results), "failed": len(failed),
        "output_tokens": n_tok, "makespan_s": round(t_end - t0, 3),
        "output_tokens_per_s": round(n_tok / (t_end - t0), 1),
        "ttft_ms": {"p50": round(_pct(ttft, 0.5), 1), "p90": round(_pct(ttft, 0.9), 1),
                    "max": round(max(ttft), 1)},
        "e2e_ms": {"p50": round(_pct(e2e, 0.5), 1), "p90": round(_pct(e2e, 0.9), 1),
                   "max": round(max(e2e), 1)},
        "tpot_ms": {"p50": round(_pct(tpot, 0.5), 3), "p90": round(_pct(tpot, 0.9), 3)},
        "prefill_ms_p50": round(_pct([f["prefill_ms"] for f in firsts.values()], 0.5), 1),
        "load_ms_p50": round(_pct([results[r]["load_ms"] for r in results], 0.5), 2),
        "occupancy_p50": _pct([results[r]["occupancy"] for r in results], 0.5),
        "producers": args.producers, "batch_width": args.batch,
        # Where the time to first token goes: waiting for a producer (its
        # earlier prompts) and the prefill itself.
        "ttft_parts_ms": {
            "queued_p50": round(_pct(queued, 0.5), 1), "queued_p90": round(_pct(queued, 0.9), 1),
            "prefill_p50": round(_pct([f["prefill_ms"] for f in firsts.values()], 0.5), 1),
            "prefill_p90": round(_pct([f["prefill_ms"] for f in firsts.values()], 0.9), 1)},
        "decode_step_ms": {"steps": len(step_ms), "p50": round(_pct(step_ms, 0.5), 3),
                           "p90": round(_pct(step_ms, 0.9), 3),
                           "p99": round(_pct(step_ms, 0.99), 3), "max": round(max(step_ms), 3)}
        if step_ms else {},
        "decode_steps_by_overlapping_prefills": contention(
            steps, [(f["t0"], f["t"]) for f in firsts.values()], t0, t_end),
    }
    return summary, {r: results[r]["tokens"] for r in results}


def run(args):
    """Start the children, feed the workload at its arrival times (``repeats``
    passes, each with request ids of its own), collect results."""
    root = tempfile.mkdtemp(prefix="pd1gpu-", dir="/dev/shm" if os.path.isdir("/dev/shm") else None)
    env = dict(os.environ, PD_SHM_ROOT=root, PD_KV_PULL_TIMEOUT=str(args.timeout),
               PYTHONPATH=os.path.dirname(os.path.dirname(os.path.dirname(
                   os.path.abspath(__file__)))))
    events = queue.Queue()
    names = ["consumer"] + [f"producer{i}" for i in range(args.producers)]
    procs = {n: _child("consumer" if n == "consumer" else "producer", args, root, env)
             for n in names}
    for n, p in procs.items():
        threading.Thread(target=_pump, args=(n, p, events), daemon=True).start()
    passes, tokens = [], {}
    try:
        ready = set()
        deadline = time.monotonic() + args.timeout * 4
        while len(ready) < len(procs):
            n, ev = events.get(timeout=max(1.0, deadline - time.monotonic()))
            if ev["ev"] == "ready":
                ready.add(n)
                _log(f"{n} ready")
            elif ev["ev"] == "eof":
                raise RuntimeError(f"{n} exited before it was ready")
        for rep in range(args.repeats):
            summary, toks = _pass(args, rep, procs, names, events)
            passes.append(summary)
            tokens.update(toks)
            _log(f"pass {rep}: {summary['output_tokens_per_s']} tok/s, TTFT p50 "
                 f"{summary['ttft_ms']['p50']} ms, TPOT p50 {summary['tpot_ms']['p50']} ms")
    finally:
        for p in procs.values():
            try:
                p.stdin.write(json.dumps({"cmd": "stop"}) + "\n")
                p.stdin.flush()
            except (BrokenPipeError, ValueError):
                pass
        for n, p in procs.items():
            try:
                p.wait(timeout=args.timeout)
            except subprocess.TimeoutExpired:
                p.kill()
                p.wait()
        shutil.rmtree(root, ignore_errors=True)
    bad = [n for n, p in procs.items() if p.returncode != 0]
    if bad:
        raise RuntimeError(f"children exited with errors: {bad}")
    summary = dict(passes[0])
    if len(passes) > 1:
        spread = lambda f: [f(x) for x in passes]   # noqa: E731
        summary["passes"] = passes
        summary["across_passes"] = {
            "output_tokens_per_s": spread(lambda x: x["output_tokens_per_s"]),
            "ttft_p50_ms": spread(lambda x: x["ttft_ms"]["p50"]),
            "tpot_p50_ms": spread(lambda x: x["tpot_ms"]["p50"]),
            "tpot_p90_ms": spread(lambda x: x["tpot_ms"]["p90"])}
    return summary, tokens


def parse(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("role", choices=["run", "producer", "consumer", "control"])
    ap.add_argument("--root", default=None)
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--requests", type=int, default=64)
    ap.add_argument("--rate", type=float, default=20.0)
    ap.add_argument("--min-len", type=int, default=128)
    ap.add_argument("--max-len", type=int, default=1024)
    ap.add_argument("--max-new", type=int, default=128)
    ap.add_argument("--batch", type=int, default=16)
    ap.add_argument("--producers", type=int, default=2)
    ap.add_argument("--ipc-slots", type=int, default=8)
    ap.add_argument("--layers", type=int, default=0)
    ap.add_argument("--small", action="store_true", help="a 2-layer test-size model")
    ap.add_argument("--eager", action="store_true", help="decode without HIP graphs")
    ap.add_argument("--timeout", type=float, default=120.0)
    ap.add_argument("--tokens-out", default=None, help="write each request's tokens (JSON)")
    ap.add_argument("--repeats", type=int, default=1,
                    help="passes of the same workload in one run (children stay up)")
    ap.add_argument("--plan-batch", type=int, default=16,
                    help="batch size the decode attention plans its context split for (the "
                         "consumer and the control use max(--batch, this)): equal values give "
                         "each request the same tokens whatever batches it shares")
    return ap.parse_args(argv)


def main(argv=None):
    args = parse(argv)
    if args.role == "producer":
        producer(args)
    elif args.role == "consumer":
        consumer(args)
    elif args.role == "control":
        control(args)
    else:
        summary, tokens = run(args)
        if args.tokens_out:
            with open(args.tokens_out, "w") as f:
                json.dump(tokens, f)
        print(json.dumps(summary), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
