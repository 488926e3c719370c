"""Continuous scheduling and prefetch semantics on the CPU, with a stand-in decoder.

The decoder's next token is a fixed function of (token, ctx), so every
stream's output is known in advance; the cache is a real PagedKVCache on the
CPU (block bookkeeping only). Follows the behaviours of _ContinuousScheduler
(serving/cluster.py:832-1134) and DecodeWorkerBase.prefetch (:350-436).
"""
import threading
import time

import pytest
import torch

from rngd_pd_amd.engines.paged_cache import PagedKVCache
from rngd_pd_amd.serving.scheduler import ContinuousScheduler, Prefetcher


def nxt(tok, ctx):
    return (tok * 7 + ctx) % 101


class FakeDecoder:
    def __init__(self, B, fail_at=None, delay=0.0):
        self.tokens = torch.zeros(B, dtype=torch.int32)
        self.calls, self.fail_at, self.max_live = [], fail_at, 0
        self.delay = delay

    def step(self, tok, ctx, tab, max_ctx):
        if self.delay:
            time.sleep(self.delay)
        self.calls.append((tok.tolist(), ctx.tolist(), tab.clone()))
        self.max_live = max(self.max_live, tok.numel())
        if self.fail_at is not None and len(self.calls) == self.fail_at:
            raise RuntimeError("step failed")
        out = [nxt(int(t), int(c)) for t, c in zip(tok.tolist(), ctx.tolist())]
        self.tokens[:len(out)] = torch.tensor(out, dtype=torch.int32)
        return self.tokens[:len(out)]


def expected(first, pos, max_new):
    outs, cur = [first], first
    while len(outs) < max_new:
        cur = nxt(cur, pos + 1)
        outs.append(cur)
        pos += 1
    return outs


def make(B=2, blocks=256, fail_at=None, delay=0.0, **kw):
    cache = PagedKVCache(1, blocks, 1, 32, device="cpu")
    dec = FakeDecoder(B, fail_at, delay)
    prompts = {}

    def produce(item):
        if item.get("gate") is not None:
            item["gate"].wait(5)
        if item.get("bad"):
            raise IOError(f"load of {item['req_id']} failed")
        P = item["P"]
        cache.allocate(item["req_id"], P)
        prompts[item["req_id"]] = P
        return item["first"], P, 1.0

    sch = ContinuousScheduler(B, dec, cache, produce, use_graphs=False, device="cpu", **kw)
    return sch, dec, cache


def test_streams_follow_their_own_positions_and_free_blocks():
    sch, dec, cache = make(B=2)
    reqs = [dict(req_id=f"r{i}", P=P, first=f, max_new=n)
            for i, (P, f, n) in enumerate([(5, 3, 6), (17, 9, 3), (31, 4, 9), (1, 0, 1), (16, 50, 4)])]
    items = [sch.submit_async(r) for r in reqs]
    for it in items:
        assert it["ev"].wait(10)
        assert it["err"] is None
        assert it["out"]["tokens"] == expected(it["first"], it["P"], it["max_new"])
        assert it["out"]["pos"] == it["P"]
    assert dec.max_live <= 2
    assert cache.alloc.free_blocks() == 256                 # every block came back
    sch.close()


def test_step_inputs_carry_ctx_and_block_tables():
    sch, dec, cache = make(B=4)
    seen = {}
    orig = dec.step

    def spy(tok, ctx, tab, max_ctx):
        for row, c in enumerate(ctx.tolist()):
            seen.setdefault(c, tab[row].tolist())
        return orig(tok, ctx, tab, max_ctx)
    dec.step = spy
    out = sch.submit(dict(req_id="a", P=15, first=1, max_new=4))   # positions 15, 16, 17
    assert out["tokens"] == expected(1, 15, 4)
    assert sorted(seen) == [16, 17, 18]
    assert sum(b >= 0 for b in seen[16]) == 1 and sum(b >= 0 for b in seen[17]) == 2
    sch.close()


def test_failed_load_fails_only_its_request():
    sch, _dec, _cache = make(B=2)
    good = sch.submit_async(dict(req_id="g", P=4, first=2, max_new=5))
    bad = sch.submit_async(dict(req_id="b", P=4, first=2, max_new=5, bad=True))
    assert bad["ev"].wait(10) and isinstance(bad["err"], IOError)
    assert good["ev"].wait(10) and good["err"] is None
    with pytest.raises(IOError):
        sch.submit(dict(req_id="b2", P=4, first=2, max_new=5, bad=True))
    sch.close()


def test_failed_step_fails_the_batch_and_the_loop_goes_on():
    sch, _dec, cache = make(B=2, fail_at=2)
    a = sch.submit_async(dict(req_id="a", P=4, first=2, max_new=6))
    assert a["ev"].wait(10) and isinstance(a["err"], RuntimeError)
    out = sch.submit(dict(req_id="c", P=8, first=5, max_new=3))
    assert out["tokens"] == expected(5, 8, 3)
    assert cache.alloc.free_blocks() == 256
    sch.close()


def test_request_longer_than_the_table_fails_alone():
    sch, _dec, _cache = make(B=2, max_blocks=2)              # 32 tokens per stream
    it = sch.submit_async(dict(req_id="long", P=30, first=1, max_new=5))
    assert it["ev"].wait(10) and isinstance(it["err"], ValueError)
    assert sch.submit(dict(req_id="ok", P=20, first=1, max_new=5))["tokens"] == expected(1, 20, 5)
    sch.close()


def test_admit_min_holds_lanes_and_counts_them():
    """With a stream running and admit_min=2, one ready request waits (held)
    until a second is ready too; lanes with nothing waiting count as starved."""
    sch, dec, _cache = make(B=4, admit_min=2, delay=0.002)
    gate = threading.Event()
    first = sch.submit_async(dict(req_id="run", P=4, first=1, max_new=200))
    time.sleep(0.05)
    one = sch.submit_async(dict(req_id="one", P=4, first=1, max_new=3))
    time.sleep(0.05)
    two = sch.submit_async(dict(req_id="two", P=4, first=1, max_new=3, gate=gate))
    time.sleep(0.05)
    gate.set()
    for it in (first, one, two):
        assert it["ev"].wait(10) and it["err"] is None
    assert sch.held_lane_steps > 0 and sch.starved_lane_steps > 0
    assert first["out"]["occupancy"] > 0
    sch.close()


def test_prefetch_cap_ttl_and_join():
    started = threading.Event()
    release = threading.Event()
    loads = []

    def load(req):
        loads.append(req)
        if req == "slow":
            started.set()
            release.wait(5)
        return f"kv:{req}"

    p = Prefetcher(load, cap=2, ttl_s=900)
    assert p.prefetch("slow") == {"prefetch": "started", "req_id": "slow"}
    assert p.prefetch("slow") == {"prefetch": "already running"}
    assert p.prefetch("b")["prefetch"] == "started"
    assert p.prefetch("c") == {"prefetch": "skipped (full)", "req_id": "c"}
    assert started.wait(5)
    release.set()
    res, lead = p.take("slow")
    assert res == "kv:slow" and lead >= 0
    res, lead = p.take("c")                                   # never prefetched: loads now
    assert res == "kv:c" and lead == -1.0
    p.ttl_s = 0.0                                             # everything left is stale
    assert p.prefetch("d")["prefetch"] == "started"           # "b" reclaimed, not counted
    assert p.outstanding() == ["d"]


def test_contention_groups_steps_by_overlapping_prefills():
    """Config-5 diagnosis: each decode step is counted with the number of
    prefills whose [start, end) overlaps it, inside the pass window only."""
    from rngd_pd_amd.serving.pd_one_gpu import contention
    prefills = [(10.0, 10.1), (10.05, 10.2)]
    steps = [
        (9.0, 5.0, 4),        # before the pass window: ignored
        (10.0, 4.0, 4),       # [10.000, 10.004): overlaps the first prefill
        (10.06, 6.0, 4),      # [10.060, 10.066): both
        (10.15, 5.0, 4),      # [10.150, 10.155): the second
        (10.3, 3.0, 4),       # after both
        (10.31, 3.5, 4),
    ]
    got = contention(steps, prefills, 9.5, 11.0)
    assert got["0_prefills"] == {"steps": 2, "step_ms_p50": 3.5, "step_ms_p90": 3.5}
    assert got["1_prefills"]["steps"] == 2
    assert got["2_prefills"] == {"steps": 1, "step_ms_p50": 6.0, "step_ms_p90": 6.0}


def test_step_log_is_taken_and_cleared():
    from rngd_pd_amd.serving.scheduler import ContinuousScheduler
    sched = ContinuousScheduler.__new__(ContinuousScheduler)
    sched.step_log = [(1.0, 2.0, 3)]
    sched._log_lock = threading.Lock()
    assert sched.take_step_log() == [(1.0, 2.0, 3)]
    assert sched.take_step_log() == []


def test_each_pass_replays_the_workload_under_its_own_ids():
    from rngd_pd_amd.serving.pd_one_gpu import parse, workload
    args = parse(["run", "--requests", "5", "--small"])
    a, b = workload(args, 0), workload(args, 2)
    assert [r["req"] for r in a] == [f"q{i}" for i in range(5)]
    assert [r["req"] for r in b] == [f"r2q{i}" for i in range(5)]
    assert [(r["arrival"], r["tokens"]) for r in a] == [(r["arrival"], r["tokens"]) for r in b]
