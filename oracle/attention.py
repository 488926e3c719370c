"""numpy restatement of the reference's decode attention -- TEST INFRASTRUCTURE.

cpu_attention follows the attention lines of cpu_layer
(kernels/decode_batch.py:147-156) on the reference's dense per-stream layout:
K [B, NKV, HD, S], V [B, NKV, S, HD]. The paged conversions are plain numpy
indexing, written independently of the C oracle, so the two check each other.
"""
import math

import numpy as np


def cpu_attention(q, K, V, positions, k_new=None, v_new=None):
    """q float32 [B, NH, HD] (after RoPE, unscaled); K/V dense layout.

    Writes k_new/v_new [B, NKV, HD] at positions[b] when given (:147-150),
    scores q.K / sqrt(HD) (:151), slots > pos set to -1e4 (:152-153),
    max-subtracted softmax (:154-155), p.V (:156). Returns [B, NH, HD]."""
    B, NH, HD = q.shape
    NKV = K.shape[1]
    G = NH // NKV
    K, V = K.copy(), V.copy()
    if k_new is not None:
        for b in range(B):
            K[b, :, :, positions[b]] = k_new[b]
            V[b, :, positions[b], :] = v_new[b]
    sc = np.einsum("bkgh,bkhs->bkgs", q.reshape(B, NKV, G, HD), K) / math.sqrt(HD)
    for b in range(B):
        sc[b, :, :, positions[b] + 1:] = -1e4
    sc = sc - sc.max(-1, keepdims=True)
    p = np.exp(sc)
    p /= p.sum(-1, keepdims=True)
    return np.einsum("bkgs,bksh->bkgh", p, V).reshape(B, NH, HD)


def k_block_index(D):
    """int64 [16, D]: element offset of (token slot, dim) inside one K block of
    the paged cache (16 tokens x D dims, D % 32 == 0).

    The block is 16-byte units of 8 consecutive dims of one token; the unit of
    (slot, d // 8) is ((t * (D // 32) + d // 32) * 4 + (d // 8) % 4) * 8 + j8
    with t = (slot >> 2) & 1 and j8 = (slot >> 3) * 4 + (slot & 3). This is a
    layout of this package's paged cache, not of the reference (whose decode K is dense
    [nl, B, NKV, HD, S], engines/decode_batch.py:305-330)."""
    if D % 32:
        raise ValueError(f"head_dim {D} is not a multiple of 32")
    slot = np.arange(16)[:, None]
    d = np.arange(D)[None, :]
    t = (slot >> 2) & 1
    j8 = (slot >> 3) * 4 + (slot & 3)
    unit = ((t * (D // 32) + d // 32) * 4 + (d // 8) % 4) * 8 + j8
    return (unit * 8 + d % 8).astype(np.int64)


def k_block_rows(ck):
    """Paged K blocks [..., 16, D] (tiled) -> token rows [..., 16, D]."""
    D = ck.shape[-1]
    flat = np.ascontiguousarray(ck).reshape(ck.shape[:-2] + (16 * D,))
    return flat[..., k_block_index(D)]


def k_block_tiled(rows):
    """Token rows [..., 16, D] -> paged K blocks [..., 16, D] (tiled)."""
    D = rows.shape[-1]
    out = np.empty(rows.shape[:-2] + (16 * D,), rows.dtype)
    out[..., k_block_index(D)] = rows
    return out.reshape(rows.shape)


def paged_from_dense(K, V, ctx, tables, num_blocks, bs=16):
    """Dense per-stream caches -> one layer of the paged cache.

    K [B, H, D, S], V [B, H, S, D] (any dtype); tables int [B, max_blocks].
    Returns cache_k [nb, H, bs, D] (tiled blocks, k_block_index), cache_v
    [nb, H, D, bs] holding tokens 0..ctx[b]-1 of each stream (zeros elsewhere)."""
    B, H, D, S = K.shape
    rows = np.zeros((num_blocks, H, bs, D), K.dtype)
    cv = np.zeros((num_blocks, H, D, bs), V.dtype)
    for b in range(B):
        for t in range(ctx[b]):
            blk, slot = tables[b][t // bs], t % bs
            rows[blk, :, slot, :] = K[b, :, :, t]
            cv[blk, :, :, slot] = V[b, :, t, :]
    return k_block_tiled(rows), cv
