"""Paged decode-side KV cache and its block allocator.

Replaces the reference's per-stream S-wide lanes ([nl, B, NKV, HD, S] /
[nl, B, NKV, S, HD], engines/decode_batch.py:305-330) with fixed 16-token
blocks shared by every request: a request holds ceil(tokens/16) blocks in any
order, listed in its block table (the same table for every layer). Capacity
is then set by HBM, not by a compiled S.

Layout (bf16): K [L, num_blocks, Hkv, 16, D] and V [L, num_blocks, Hkv, D, 16]
(dim rows, contiguous tokens). A K block holds its 16 tokens x D dims as
16-byte units of 8 dims of one token, tiled in the order the decode-attention
QK tiles read them (k_block_index); V is already in the order the PV tiles
read. k_block_rows / k_block_tiled convert K blocks to and from token rows.
"""
import threading

import numpy as np
import torch

from ..kernels import handoff as _h

BLOCK = 16


def k_block_index(head_dim, device=None):
    """int64 [16, head_dim]: position of (token slot, dim) inside one K block.

    Unit (16 bytes, 8 dims) of slot s and dims d0..d0+7 is
    ((t * head_dim/32 + d0/32) * 4 + (d0/8) % 4) * 8 + j8 with t = bit 2 of s
    and j8 = (s // 8) * 4 + s % 4 -- the order of rngdpd.h's paged cache."""
    if head_dim % 32:
        raise ValueError(f"head_dim {head_dim} is not a multiple of 32")
    s = torch.arange(BLOCK, device=device).view(BLOCK, 1)
    d = torch.arange(head_dim, device=device).view(1, head_dim)
    unit = ((((s >> 2) & 1) * (head_dim // 32) + d // 32) * 4 + (d // 8) % 4) * 8 \
        + (s >> 3) * 4 + (s & 3)
    return unit * 8 + d % 8


def k_block_rows(blocks):
    """K blocks [..., 16, D] in cache order -> token rows [..., 16, D]."""
    D = blocks.shape[-1]
    flat = blocks.reshape(*blocks.shape[:-2], BLOCK * D)
    return flat[..., k_block_index(D, blocks.device)]


def k_block_tiled(rows):
    """Token rows [..., 16, D] -> K blocks [..., 16, D] in cache order."""
    D = rows.shape[-1]
    out = torch.empty(*rows.shape[:-2], BLOCK * D, dtype=rows.dtype, device=rows.device)
    out[..., k_block_index(D, rows.device).reshape(-1)] = rows.reshape(*rows.shape[:-2], BLOCK * D)
    return out.view(rows.shape)


class BlockAllocator:
    """Free list of block ids. ``seed`` shuffles the initial order (a permuted
    block table, as the handoff workloads use)."""

    def __init__(self, num_blocks, seed=None):
        ids = np.arange(num_blocks, dtype=np.int64)
        if seed is not None:
            ids = np.random.default_rng(seed).permutation(num_blocks)
        self._free = [int(i) for i in ids[::-1]]
        self.num_blocks = num_blocks
        self._lock = threading.Lock()

    def free_blocks(self):
        return len(self._free)

    def allocate(self, n):
        with self._lock:
            if n > len(self._free):
                raise MemoryError(f"paged cache exhausted: need {n} blocks, {len(self._free)} free")
            return [self._free.pop() for _ in range(n)]

    def release(self, blocks):
        with self._lock:
            self._free.extend(reversed(list(blocks)))


class PagedKVCache:
    """One paged K/V cache for all layers plus per-request block tables."""

    def __init__(self, n_layers, num_blocks, n_kv_heads=8, head_dim=128, device="cuda",
                 seed=None, dtype=torch.bfloat16):
        self.n_layers, self.num_blocks = n_layers, num_blocks
        self.n_kv_heads, self.head_dim = n_kv_heads, head_dim
        self.device = torch.device(device)
        self.k = torch.zeros((n_layers, num_blocks, n_kv_heads, BLOCK, head_dim), dtype=dtype,
                             device=self.device)
        self.v = torch.zeros((n_layers, num_blocks, n_kv_heads, head_dim, BLOCK), dtype=dtype,
                             device=self.device)
        self.alloc = BlockAllocator(num_blocks, seed)
        self._tables = {}          # req_id -> [block ids]
        self._dev_tables = {}      # req_id -> device int32 tensor
        self._lock = threading.Lock()

    # -- block tables ---------------------------------------------------------
    def allocate(self, req_id, n_tokens):
        """Blocks for the first ``n_tokens`` tokens of a new request."""
        need = (n_tokens + BLOCK - 1) // BLOCK
        with self._lock:
            if req_id in self._tables:
                raise KeyError(f"request {req_id!r} already holds blocks")
            self._tables[req_id] = self.alloc.allocate(need)
            self._dev_tables.pop(req_id, None)
        return self.table(req_id)

    def ensure(self, req_id, n_tokens):
        """Grow the request's table to cover ``n_tokens`` tokens (decode growth)."""
        need = (n_tokens + BLOCK - 1) // BLOCK
        with self._lock:
            have = self._tables.setdefault(req_id, [])
            if need > len(have):
                have.extend(self.alloc.allocate(need - len(have)))
                self._dev_tables.pop(req_id, None)

    def free(self, req_id):
        with self._lock:
            blocks = self._tables.pop(req_id, [])
            self._dev_tables.pop(req_id, None)
        self.alloc.release(blocks)

    def blocks(self, req_id):
        return list(self._tables[req_id])

    def table(self, req_id):
        """Device int32 block table of the request."""
        with self._lock:
            t = self._dev_tables.get(req_id)
            if t is None:
                t = torch.tensor(self._tables[req_id] or [0], dtype=torch.int32, device=self.device)
                self._dev_tables[req_id] = t
            return t

    def batch_tables(self, req_ids, max_blocks=None):
        """[B, max_blocks] device int32 tables (unused entries -1)."""
        rows = [self._tables[r] for r in req_ids]
        width = max_blocks or max(1, max(len(r) for r in rows))
        arr = np.full((len(rows), width), -1, np.int32)
        for i, r in enumerate(rows):
            arr[i, :len(r)] = r
        return torch.from_numpy(arr).to(self.device)

    # -- frames in and out ----------------------------------------------------
    def write_frame(self, req_id, frame, num_tokens, S, stream=None):
        """Scatter tokens 0..num_tokens-1 of a transport frame [L, 2, Hkv*D*S]."""
        _h.scatter_paged(frame, self.table(req_id), num_tokens, S, self.k, self.v, stream=stream)

    def read_frame(self, req_id, num_tokens, S, frame=None, stream=None):
        """The request's S-wide transport frame (zero for t >= num_tokens)."""
        return _h.gather_paged(self.k, self.v, self.table(req_id), num_tokens, S, frame=frame,
                               stream=stream)

    def view(self, req_id, num_tokens, S):
        """What the connector's decode side registers for one request."""
        return PagedRequestView(self, req_id, num_tokens, S)


class PagedRequestView:
    """One request's slice of a PagedKVCache, as registered with the connector."""

    def __init__(self, cache, req_id, num_tokens, S):
        self.cache, self.req_id = cache, req_id
        self.num_tokens, self.S = num_tokens, S
        if req_id not in cache._tables:
            cache.allocate(req_id, num_tokens)

    @property
    def table(self):
        return self.cache.table(self.req_id)
