"""Prefill, and prefill/decode disaggregation on one GPU.

* LlamaPrefill against the oracle (oracle/decode.py, pinned to transformers'
  Llama): the prompt's K/V per layer and the first token.
* The 2-producer / 1-consumer run (rngd_pd_amd.serving.pd_one_gpu): every
  request completes, and its greedy tokens equal those of a one-process
  control that prefills and decodes the same prompts with the same weights,
  one request at a time. The decode step is batch-invariant: every kernel
  computes a stream's row independently of the others, and attention plans
  its context split for a fixed plan batch, not for the streams present. So
  continuous batching, admission order and the handoff must not change a
  single token. Checked on a small model at widths 1 and 4, and at the
  Llama-3.1-8B shape (random-init weights, 32 layers) at width 16 with
  prompts of 128 to 1024 tokens.
"""
import json
import os
import subprocess
import sys

import numpy as np
import pytest
import torch

from oracle import decode as od

pytestmark = pytest.mark.gpu

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_prefill_matches_oracle(cuda):
    from rngd_pd_amd.engines.llama_decode import LlamaConfig, LlamaWeights
    from rngd_pd_amd.engines.llama_prefill import LlamaPrefill
    cfg = LlamaConfig(hidden=512, n_heads=8, n_kv_heads=2, head_dim=128, inter=1024,
                      vocab=1000, n_layers=2)
    w = LlamaWeights.random(cfg, seed=4, device=cuda)
    pre = LlamaPrefill(w)
    rng = np.random.default_rng(4)
    f = lambda t: t.float().cpu().numpy()   # noqa: E731
    T_ = lambda t: np.ascontiguousarray(f(t).T)   # noqa: E731
    ow = {"embed": f(w.embed), "norm_f": f(w.norm_f), "lm_head": T_(w.lm_head),
          "layers": [(f(w.norm1[i]), T_(w.wqkv[i]), T_(w.wo[i]), f(w.norm2[i]), T_(w.wgu[i]),
                      T_(w.wd[i])) for i in range(cfg.n_layers)]}

    class C:
        n_heads, n_kv_heads, eps = cfg.n_heads, cfg.n_kv_heads, cfg.eps
        inv = cfg.inv_freq().numpy()

    for T in (1, 37, 130):
        tokens = rng.integers(0, cfg.vocab, T)
        print(f"prefill T={T}", flush=True)
        first, k, v = pre.forward(tokens)
        torch.cuda.synchronize()
        Ks = [np.zeros((1, cfg.n_kv_heads, T, cfg.head_dim), np.float32) for _ in range(2)]
        Vs = [np.zeros((1, cfg.n_kv_heads, T, cfg.head_dim), np.float32) for _ in range(2)]
        for t in range(T):
            tok, _x, logits = od.decode_step(tokens[t:t + 1], ow, Ks, Vs, [t], C)
        for li in range(cfg.n_layers):
            got_k = k[li].float().cpu().numpy().transpose(1, 0, 2)     # [Hkv, T, D]
            got_v = v[li].float().cpu().numpy().transpose(1, 0, 2)
            assert od.rel_l2(got_k, Ks[li][0]) < 0.02, (T, li)
            assert od.rel_l2(got_v, Vs[li][0]) < 0.02, (T, li)
        top2 = np.sort(logits[0])[-2:]
        if top2[1] - top2[0] > 0.05 * np.abs(logits[0]).max():
            assert first == int(tok[0]), T


def _run(args):
    env = dict(os.environ, PYTHONPATH=REPO)
    cmd = [sys.executable, "-u", "-m", "rngd_pd_amd.serving.pd_one_gpu"] + args
    print("running", " ".join(args), flush=True)
    r = subprocess.run(cmd, env=env, cwd=REPO, stdout=subprocess.PIPE, stderr=subprocess.STDOUT,
                       text=True, timeout=300)
    assert r.returncode == 0, r.stdout[-4000:]
    return r.stdout


COMMON = ["--small", "--requests", "6", "--rate", "40", "--min-len", "20", "--max-len", "200",
          "--max-new", "12", "--seed", "3"]


def test_two_producers_one_consumer_match_control(tmp_path):
    out = _run(["control"] + COMMON)
    want = {}
    for line in out.splitlines():
        if line.startswith("{"):
            ev = json.loads(line)
            want[ev["req"]] = ev["tokens"]
    assert len(want) == 6 and all(len(t) == 12 for t in want.values())
    for batch in (1, 4):
        tok_file = tmp_path / f"tokens_b{batch}.json"
        out = _run(["run", "--batch", str(batch), "--tokens-out", str(tok_file)] + COMMON)
        summary = json.loads([ln for ln in out.splitlines() if ln.startswith("{")][-1])
        print(f"batch {batch}: {summary}", flush=True)
        assert summary["completed"] == 6 and summary["failed"] == 0
        got = json.loads(tok_file.read_text())
        assert got == want, f"batch {batch}: tokens differ from the one-process control"


def test_repeated_passes_give_the_same_tokens(tmp_path):
    """Passes of one run replay the workload on the same processes: every
    pass's tokens equal the control's, and each pass reports its decode steps
    grouped by overlapping prefills (the config-5 spread diagnosis)."""
    out = _run(["control"] + COMMON)
    want = {}
    for line in out.splitlines():
        if line.startswith("{"):
            ev = json.loads(line)
            want[ev["req"]] = ev["tokens"]
    tok_file = tmp_path / "tokens.json"
    out = _run(["run", "--batch", "4", "--repeats", "2", "--tokens-out", str(tok_file)] + COMMON)
    summary = json.loads([ln for ln in out.splitlines() if ln.startswith("{")][-1])
    assert len(summary["passes"]) == 2
    for p in summary["passes"]:
        assert p["completed"] == 6 and p["failed"] == 0
        groups = p["decode_steps_by_overlapping_prefills"]
        assert sum(g["steps"] for g in groups.values()) == p["decode_step_ms"]["steps"] > 0
        assert p["ttft_parts_ms"]["queued_p50"] >= 0
    got = json.loads(tok_file.read_text())
    assert len(got) == 12
    for req, toks in want.items():
        assert got[req] == toks and got["r1" + req] == toks, req


def test_llama8b_two_producers_one_consumer_match_control(tmp_path):
    """The serving workload's shape: Llama-3.1-8B, two prefill producer processes
    and one decode consumer at width 16 on this GPU, Poisson arrivals, prompts
    U[128, 1024]; fewer requests and output tokens than the benchmark run so
    the control (one request at a time) stays short."""
    common = ["--requests", "24", "--rate", "40", "--min-len", "128", "--max-len", "1024",
              "--max-new", "24", "--seed", "5"]
    out = _run(["control"] + common)
    want = {}
    for line in out.splitlines():
        if line.startswith("{"):
            ev = json.loads(line)
            want[ev["req"]] = ev["tokens"]
    assert len(want) == 24 and all(len(t) == 24 for t in want.values())
    tok_file = tmp_path / "tokens_8b.json"
    out = _run(["run", "--batch", "16", "--producers", "2", "--tokens-out", str(tok_file)] + common)
    summary = json.loads([ln for ln in out.splitlines() if ln.startswith("{")][-1])
    print(f"llama-8b 2P:1D: {summary}", flush=True)
    assert summary["completed"] == 24 and summary["failed"] == 0
    got = json.loads(tok_file.read_text())
    diff = [r for r in want if got.get(r) != want[r]]
    assert not diff, f"{len(diff)} requests' tokens differ from the control: {diff[:4]}"
