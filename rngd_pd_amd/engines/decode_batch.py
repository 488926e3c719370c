"""Batched decode attention over the paged cache (the consumer of the handoff).

The attention part of the reference's BatchDecodeEngine step
(engines/decode_batch.py:422-442 -> kernels/decode_batch.py:81-85) with its
position semantics (serving/cluster.py:1242-1264, engines/decode_batch.py:246-261):
a stream whose prompt held P tokens decodes its first token at position P;
at position pos the new token's k/v are written to slot pos (the reference's
one-hot injection) and attention covers slots 0..pos. Query head h reads KV
head h // (Hq / Hkv). The 1/sqrt(D) scale is applied in the kernel unless the
caller folds it into q (scale=1.0, as the reference folds it into wq).

Admission is a frame scatter into freshly allocated blocks, the paged form of
write_slot_kv (engines/decode_batch.py:357-377); retirement frees the blocks.
"""
import math

import torch

from ..kernels import attention as _attn
from .paged_cache import PagedKVCache


class BatchDecodeAttention:
    """Decode attention for a batch of streams sharing one PagedKVCache."""

    def __init__(self, cache: PagedKVCache, n_q_heads=32, scale=None):
        self.cache = cache
        self.Hq = n_q_heads
        self.G = n_q_heads // cache.n_kv_heads
        self.scale = (1.0 / math.sqrt(cache.head_dim)) if scale is None else scale
        self.positions = {}                  # req_id -> next decode position
        self._batch_key = None
        self._tables = None
        self._ws = None

    def admit(self, req_id, frame, num_tokens, S, stream=None):
        """Place a handed-off request: its S-wide frame, first decode position num_tokens."""
        if req_id not in self.cache._tables:
            self.cache.allocate(req_id, num_tokens + 1)
        self.cache.write_frame(req_id, frame, num_tokens, S, stream=stream)
        self.positions[req_id] = num_tokens
        self._batch_key = None

    def admit_loaded(self, req_id, num_tokens):
        """A request the connector already scattered (register_kv_caches path)."""
        self.cache.ensure(req_id, num_tokens + 1)
        self.positions[req_id] = num_tokens
        self._batch_key = None

    def retire(self, req_id):
        self.positions.pop(req_id, None)
        self.cache.free(req_id)
        self._batch_key = None

    def prepare(self, req_ids):
        """Block tables and context lengths for one step of ``req_ids`` (growing
        each stream's blocks to hold its new token)."""
        for r in req_ids:
            self.cache.ensure(r, self.positions[r] + 1)
        key = (tuple(req_ids), tuple(len(self.cache._tables[r]) for r in req_ids))
        if key != self._batch_key:
            self._tables = self.cache.batch_tables(req_ids)
            self._batch_key = key
        pos = [self.positions[r] for r in req_ids]
        ctx = torch.tensor([p + 1 for p in pos], dtype=torch.int32, device=self.cache.device)
        return self._tables, ctx, max(pos) + 1

    def layer_attention(self, layer, q, k_new, v_new, tables, ctx, max_ctx, out=None, stream=None):
        """One layer: write the new token's k/v at slot pos, attend over 0..pos.
        q [B, Hq, D], k_new/v_new [B, Hkv, D] bf16 on the device."""
        ck, cv = self.cache.k[layer], self.cache.v[layer]
        _attn.cache_append(k_new, v_new, ck, cv, tables, ctx, stream=stream)
        need = _attn.workspace_bytes(q.shape[0], self.Hq, max_ctx, self.cache.head_dim)
        if need and (self._ws is None or self._ws.numel() * 4 < need):
            self._ws = torch.zeros(need // 4 + 64, dtype=torch.float32, device=self.cache.device)
        return _attn.decode_attention(q, ck, cv, tables, ctx, max_ctx, scale=self.scale, out=out,
                                      workspace=self._ws if need else None, stream=stream)

    def advance(self, req_ids):
        """After all layers of a step: every stream moves to its next position."""
        for r in req_ids:
            self.positions[r] += 1
