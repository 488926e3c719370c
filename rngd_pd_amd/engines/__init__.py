"""Decode-side engines: the paged KV cache and batched decode attention."""
