"""numpy restatement of the reference's KONI KV receiver -- TEST INFRASTRUCTURE.

Only tests use this module, as the oracle results are compared with. It follows KVReceiver.accept
(native_v4/kv.py:47-120): the same checks, in the same order, and the same
placement (tensor t = 2*layer + kind; K units land in keys[layer][h][d][tok],
V units in values[layer][h][tok][d], bf16 bits widened to float32), on dense
per-request arrays instead of the reference's lane-indexed ATOM buffers. It
handles any fragmentation by walking the concatenated frames unit by unit,
which is a different formulation from the reference's split-aware copy.
"""
import numpy as np


class ProtocolError(ValueError):
    pass


UNIT = 2048


class Receiver:
    def __init__(self, request_id, prefix_tokens, n_layers=32, n_heads=8, head_dim=128):
        self.request_id, self.n = request_id, prefix_tokens
        self.L, self.H, self.D = n_layers, n_heads, head_dim
        self.unit = n_heads * head_dim * 2
        self.keys = np.zeros((n_layers, n_heads, head_dim, prefix_tokens), np.float32)
        self.values = np.zeros((n_layers, n_heads, prefix_tokens, head_dim), np.float32)
        self.seen = np.zeros((2 * n_layers, prefix_tokens), bool)
        self.complete = False

    def accept(self, message, frames):
        """kv.py:47-120: validate the whole batch, then place it."""
        if self.complete or message.get("kind") != "kv" or message.get("request_id") != self.request_id:
            raise ProtocolError("unexpected KV message or completed request")
        entries = [{k: int(e[k]) for k in ("tier", "tensor", "block", "bytes")}
                   for e in message["entries"]]
        total = sum(e["bytes"] for e in entries)
        if not entries or total > 2 * self.L * self.n * self.unit or \
                sum(len(f) for f in frames) != total:
            raise ProtocolError("invalid payload length")
        covered = set()
        for e in entries:
            t, b, size = e["tensor"], e["block"], e["bytes"]
            if e["tier"] != 0 or not 0 <= t < 2 * self.L or size <= 0 or size % self.unit:
                raise ProtocolError("unsupported KV tensor, tier, or block size")
            if b < 0 or b + size // self.unit > self.n:
                raise ProtocolError("KV block outside admitted prefix")
            for tok in range(b, b + size // self.unit):
                if self.seen[t, tok] or (t, tok) in covered:
                    raise ProtocolError("duplicate KV block")
                covered.add((t, tok))
        if message["is_final"] and int(self.seen.sum()) + len(covered) != 2 * self.L * self.n:
            raise ProtocolError("final batch has incomplete KV coverage")
        payload = b"".join(bytes(f) for f in frames)
        off = 0
        for e in entries:
            t = e["tensor"]
            for tok in range(e["block"], e["block"] + e["bytes"] // self.unit):
                bits = np.frombuffer(payload, "<u2", self.H * self.D, off).reshape(self.H, self.D)
                off += self.unit
                val = (bits.astype(np.uint32) << 16).view(np.float32)
                if t % 2 == 0:
                    self.keys[t // 2, :, :, tok] = val
                else:
                    self.values[t // 2, :, tok, :] = val
                self.seen[t, tok] = True
        self.complete = bool(message["is_final"])
        return self.complete
