"""Writes the small golden fixtures under tests/golden/ (run from the repo root).

  wire_blobs.npz      bf16 wire blobs (the reference's pickle envelope) for a
                      (2, 3, 64) array from seed 7 and the rm-core adapter vector
                      of tests/test_airm.py:169 (seed 1, shape (2, 2, 4, 2, 8)),
                      as written by numpy 2.x.
  attention_small.npz one decode-attention case (B=2, Hq=8, Hkv=2, D=32,
                      ctx 19 and 40, permuted block tables) as dense per-stream
                      K [B, Hkv, D, S] / V [B, Hkv, S, D] bf16 bits, and its
                      output from oracle.attention.cpu_attention (the numpy
                      restatement of cpu_layer, kernels/decode_batch.py:147-156)
                      evaluated in float64.

Inputs come from numpy generators. The wire blobs come from the oracle's
pickle restatement; the attention output does not depend on the paged-cache
layout, so the test that reads it pins the C oracle's paged attention against
the dense reference formula.
"""
import math
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import attention as oatt  # noqa: E402
from oracle import wire as owire  # noqa: E402


def main():
    small = np.random.default_rng(7).standard_normal((2, 3, 64)).astype(np.float32)
    adapter = np.random.default_rng(1).standard_normal((2, 2, 4, 2, 8)).astype(np.float32)
    np.savez(os.path.join(HERE, "wire_blobs.npz"),
             small_in=small, small_blob=np.frombuffer(owire.ser(small, "bf16"), np.uint8),
             adapter_in=adapter, adapter_blob=np.frombuffer(owire.ser(adapter, "bf16"), np.uint8))

    rng = np.random.default_rng(11)
    B, Hq, H, D, S = 2, 8, 2, 32, 48
    ctx = np.array([19, 40], np.int32)
    nb = 7
    tables = np.full((B, 3), -1, np.int32)
    perm = rng.permutation(nb).astype(np.int32)
    tables[0, :2] = perm[:2]
    tables[1, :3] = perm[2:5]
    bits = lambda shape: (rng.standard_normal(shape).astype(np.float32).view(np.uint32)  # noqa: E731
                          >> 16).astype(np.uint16)
    k_dense, v_dense, q = bits((B, H, D, S)), bits((B, H, S, D)), bits((B, Hq, D))
    wide = lambda u: (u.astype(np.uint32) << 16).view(np.float32).astype(np.float64)  # noqa: E731
    out = oatt.cpu_attention(wide(q), wide(k_dense), wide(v_dense), ctx - 1).astype(np.float32)
    np.savez(os.path.join(HERE, "attention_small.npz"), q=q, k_dense=k_dense, v_dense=v_dense,
             tables=tables, ctx=ctx, scale=np.float32(1 / math.sqrt(D)), out=out)


if __name__ == "__main__":
    main()
