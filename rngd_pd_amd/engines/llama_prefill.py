"""Llama prefill for the producer side of the handoff: prompt -> per-layer KV + first token.

Stands in for FullPrefillEngine.prefill_stream (engines/prefill_full.py:337-388)
on MI355X: the prompt's K/V per layer (after RoPE, bf16, token-major
[T, Hkv, D] as the connector's device save takes them) and the greedy next
token of the last position (the reference's "next", serving/cluster.py:
330-343). Each layer's K/V is handed to ``on_layer`` as soon as the layer is
done, so saves overlap the layers that follow (the reference emits layer
groups as it goes).

Prefill is compute-bound (T tokens per weight), so its GEMMs are the
library's (hipBLASLt through torch); the norms use the decode step's RMSNorm
kernel; RoPE and causal GQA attention are fp32 torch on contiguous operands.
Activations are bf16 at tensor boundaries, as in the decode step. It takes
the decode step's LlamaWeights ([out, in] layout), so a producer and a
consumer built from one seed hold the same model.
"""
import math

import torch

from .. import _lib
from ..kernels.handoff import stream_handle

BF16 = torch.bfloat16


class LlamaPrefill:
    def __init__(self, weights, max_tokens=4096):
        self.w, self.cfg = weights, weights.cfg
        self.device = weights.embed.device
        self.max_tokens = max_tokens
        cfg = self.cfg
        self.inv = cfg.inv_freq().to(self.device)
        self.scale = 1.0 / math.sqrt(cfg.head_dim)

    def _rmsnorm(self, x, weight, out):
        T, H = x.shape
        _lib.call("pdk_rmsnorm", x.data_ptr(), None, weight.data_ptr(), T, H, self.cfg.eps,
                  out.data_ptr(), stream_handle())
        return out

    def _rope(self, t, cos, sin):
        """t [T, n, HD] bf16 -> rotate-half RoPE in fp32 -> bf16."""
        half = t.shape[-1] // 2
        f = t.float()
        a, b = f[..., :half], f[..., half:]
        return torch.cat([a * cos - b * sin, b * cos + a * sin], dim=-1).to(BF16)

    @torch.no_grad()
    def forward(self, tokens, on_layer=None, kv_out=None):
        """tokens: int sequence or int64 tensor [T] (T >= 1). Returns (first
        token, k, v) with k, v bf16 [L, T, Hkv, D] (kv_out may supply them).
        on_layer(li, k_l, v_l) is called after each layer on the current stream."""
        cfg, w, dev = self.cfg, self.w, self.device
        ids = torch.as_tensor(tokens, dtype=torch.int64, device=dev).reshape(-1)
        T = ids.numel()
        if not 1 <= T <= self.max_tokens:
            raise ValueError(f"prompt of {T} tokens outside [1, {self.max_tokens}]")
        L, H, NH, NKV, HD = cfg.n_layers, cfg.hidden, cfg.n_heads, cfg.n_kv_heads, cfg.head_dim
        G, M = NH // NKV, cfg.inter
        if kv_out is None:
            k_all = torch.empty((L, T, NKV, HD), dtype=BF16, device=dev)
            v_all = torch.empty((L, T, NKV, HD), dtype=BF16, device=dev)
        else:
            k_all, v_all = kv_out
        pos = torch.arange(T, device=dev, dtype=torch.float32)
        ang = pos[:, None] * self.inv[None, :]                     # fp32 angles, [T, HD/2]
        cos, sin = torch.cos(ang)[:, None, :], torch.sin(ang)[:, None, :]
        causal = torch.full((T, T), float("-inf"), device=dev).triu(1)
        x = w.embed.index_select(0, ids)                           # [T, H] bf16
        h = torch.empty_like(x)
        for li in range(L):
            self._rmsnorm(x, w.norm1[li], h)
            qkv = torch.nn.functional.linear(h, w.wqkv[li])         # [T, (NH + 2 NKV) HD]
            q = self._rope(qkv[:, :NH * HD].view(T, NH, HD), cos, sin)
            k = self._rope(qkv[:, NH * HD:(NH + NKV) * HD].view(T, NKV, HD), cos, sin)
            v = qkv[:, (NH + NKV) * HD:].view(T, NKV, HD)
            k_all[li].copy_(k)
            v_all[li].copy_(v)
            if on_layer is not None:
                on_layer(li, k_all[li], v_all[li])
            # Causal GQA attention in fp32: query head h reads KV head h // G.
            qf = q.float().view(T, NKV, G, HD).permute(1, 2, 0, 3).reshape(NKV, G * T, HD)
            kt = k.float().permute(1, 2, 0).contiguous()               # [NKV, HD, T]
            vf = v.float().permute(1, 0, 2).contiguous()               # [NKV, T, HD]
            sc = torch.bmm(qf.contiguous(), kt).view(NKV, G, T, T) * self.scale + causal
            p = torch.softmax(sc, dim=-1).view(NKV, G * T, T)
            ao = torch.bmm(p, vf).view(NKV, G, T, HD).permute(2, 0, 1, 3).reshape(T, NH * HD)
            x = x + torch.nn.functional.linear(ao.to(BF16), w.wo[li])
            self._rmsnorm(x, w.norm2[li], h)
            gu = torch.nn.functional.linear(h, w.wgu[li])
            act = (torch.nn.functional.silu(gu[:, :M].float()) * gu[:, M:].float()).to(BF16)
            x = x + torch.nn.functional.linear(act, w.wd[li])
        last = torch.empty((1, H), dtype=BF16, device=dev)
        self._rmsnorm(x[T - 1:T].contiguous(), w.norm_f, last)
        logits = torch.nn.functional.linear(last, w.lm_head)
        first = int(torch.argmax(logits[0]).item())
        return first, k_all, v_all
