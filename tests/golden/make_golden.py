"""Writes the small golden fixtures under tests/golden/ (run from the repo root).

  wire_blobs.npz      bf16 wire blobs (the reference's pickle envelope) for a
                      (2, 3, 64) array from seed 7 and the rm-core adapter vector
                      of tests/test_airm.py:169 (seed 1, shape (2, 2, 4, 2, 8)),
                      as written by numpy 2.x.
  attention_small.npz one decode-attention case (B=2, Hq=8, Hkv=2, D=32,
                      ctx 19 and 40, permuted blocks) and its float32 output.

Inputs come from numpy generators; the outputs from the CPU oracle, whose
functions are pinned independently in tests/test_oracle.py. The fixtures then
pin the oracle (and the numpy pickle envelope) against silent drift.
"""
import math
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import native as orc  # noqa: E402
from oracle import wire as owire  # noqa: E402


def main():
    small = np.random.default_rng(7).standard_normal((2, 3, 64)).astype(np.float32)
    adapter = np.random.default_rng(1).standard_normal((2, 2, 4, 2, 8)).astype(np.float32)
    np.savez(os.path.join(HERE, "wire_blobs.npz"),
             small_in=small, small_blob=np.frombuffer(owire.ser(small, "bf16"), np.uint8),
             adapter_in=adapter, adapter_blob=np.frombuffer(owire.ser(adapter, "bf16"), np.uint8))

    rng = np.random.default_rng(11)
    B, Hq, H, D = 2, 8, 2, 32
    ctx = np.array([19, 40], np.int32)
    nb = 7
    tables = np.full((B, 3), -1, np.int32)
    perm = rng.permutation(nb).astype(np.int32)
    tables[0, :2] = perm[:2]
    tables[1, :3] = perm[2:5]
    bits = lambda shape: (rng.standard_normal(shape).astype(np.float32).view(np.uint32)  # noqa: E731
                          >> 16).astype(np.uint16)
    ck, cv, q = bits((nb, H, 16, D)), bits((nb, H, D, 16)), bits((B, Hq, D))
    scale = 1 / math.sqrt(D)
    out = orc.decode_attn(q, ck, cv, tables, ctx, scale)
    np.savez(os.path.join(HERE, "attention_small.npz"), q=q, ck=ck, cv=cv, tables=tables,
             ctx=ctx, scale=np.float32(scale), out=out)


if __name__ == "__main__":
    main()
