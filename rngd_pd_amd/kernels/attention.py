"""torch-facing wrappers of decode attention, cache append and greedy argmax.

Replaces the attention slice of DecodeLayer.forward (kernels/decode_batch.py:81-85),
softmax_dsl (kernels/dsl_batch.py:73-86) and greedy_tokens
(engines/decode_batch.py:162-171) with HIP kernels over the paged cache.
"""
import torch

from .. import _lib
from .handoff import _need, stream_handle

BF16 = torch.bfloat16


def workspace_bytes(B, n_q_heads, max_ctx, head_dim=128):
    return int(_lib.lib().pdk_decode_attn_workspace_bytes(B, n_q_heads, max_ctx, head_dim))


_WORKSPACES = {}


def get_workspace(nbytes, device):
    """An fp32 workspace of at least ``nbytes`` on ``device``, kept per device.

    It holds the per-split partial maxima, sums and outputs of a split
    context; every entry a call reads is written earlier in that call, so one
    buffer is reused across calls without clearing. It serves one stream at a
    time: concurrent calls on different streams need their own."""
    key = torch.device(device).index or 0
    ws = _WORKSPACES.get(key)
    if ws is None or ws.numel() * 4 < nbytes:
        ws = torch.zeros(max(nbytes, 1 << 20) // 4 + 64, dtype=torch.float32, device=device)
        _WORKSPACES[key] = ws
    return ws


def _check_layer_cache(cache_k, cache_v):
    _need(cache_k, "cache_k")
    _need(cache_v, "cache_v")
    if cache_k.dim() != 4 or cache_k.shape[2] != 16:
        raise ValueError(f"cache_k must be one layer [nb, Hkv, 16, D], got {tuple(cache_k.shape)}")
    nb, H, _, D = cache_k.shape
    if tuple(cache_v.shape) != (nb, H, D, 16):
        raise ValueError(f"cache_v must be [nb, Hkv, D, 16], got {tuple(cache_v.shape)}")
    if not (cache_k.is_contiguous() and cache_v.is_contiguous()):
        raise ValueError("paged caches must be contiguous")
    return nb, H, D


def decode_attention(q, cache_k, cache_v, block_tables, ctx_lens, max_ctx, scale=1.0,
                     out=None, workspace=None, stream=None):
    """GQA decode attention for one layer.

    q [B, Hq, D] bf16 (query head h reads KV head h // (Hq/Hkv)); cache_k
    [nb, Hkv, 16, D] (tiled K blocks), cache_v [nb, Hkv, D, 16]; block_tables int32 [B, max_blocks]
    and ctx_lens int32 [B] on the device; ``max_ctx`` >= every ctx_lens[b]."""
    _need(q, "q")
    nb, H, D = _check_layer_cache(cache_k, cache_v)
    if q.dim() != 3 or q.shape[2] != D or not q.is_contiguous():
        raise ValueError(f"q must be contiguous [B, Hq, {D}], got {tuple(q.shape)}")
    B, Hq, _ = q.shape
    _need(block_tables, "block_tables", torch.int32)
    _need(ctx_lens, "ctx_lens", torch.int32)
    if block_tables.dim() != 2 or block_tables.shape[0] != B or not block_tables.is_contiguous():
        raise ValueError("block_tables must be contiguous int32 [B, max_blocks]")
    if ctx_lens.numel() != B:
        raise ValueError("ctx_lens must hold B entries")
    if out is None:
        out = torch.empty_like(q)
    need = workspace_bytes(B, Hq, max_ctx, D)
    ws = None
    if need:
        if workspace is not None:
            if workspace.numel() * workspace.element_size() < need:
                raise ValueError(f"workspace holds fewer than the {need} bytes needed")
            ws = workspace
        else:
            ws = get_workspace(need, q.device)
    ws_ptr = ws.data_ptr() if ws is not None else None
    ws_bytes = ws.numel() * ws.element_size() if ws is not None else 0
    _lib.call("pdk_decode_attn", q.data_ptr(), cache_k.data_ptr(), cache_v.data_ptr(), nb,
              block_tables.data_ptr(), block_tables.shape[1], ctx_lens.data_ptr(), int(max_ctx),
              B, Hq, H, D, float(scale), ws_ptr, ws_bytes, out.data_ptr(), stream_handle(stream))
    return out


def decode_attention_rope(qkv_partials, inv_freq, cache_k, cache_v, block_tables, ctx_lens,
                          max_ctx, n_q_heads, scale=1.0, out=None, workspace=None, stream=None,
                          plan_batch=0, ssq=None, eps=None):
    """RoPE, the new token's cache write and attention for one layer in one launch.

    qkv_partials float32 [splits, B, (n_q + 2 n_kv) D] (split-K partial sums of
    the q|k|v projection, splits in {1, 2, 4}); inv_freq float32 [D/2]. Same
    result, bit for bit, as rope_cache_append_partials then decode_attention.
    ``plan_batch`` (>= B; 0 means B) is the batch size the split plan is chosen
    for: equal plan_batch gives each stream the same result whatever B is."""
    _need(qkv_partials, "qkv_partials", torch.float32)
    _need(inv_freq, "inv_freq", torch.float32)
    nb, H, D = _check_layer_cache(cache_k, cache_v)
    if qkv_partials.dim() != 3 or not qkv_partials.is_contiguous():
        raise ValueError("qkv_partials must be contiguous [splits, B, N]")
    splits, B, N = qkv_partials.shape
    if N != (n_q_heads + 2 * H) * D:
        raise ValueError(f"qkv_partials rows hold {N} values, need {(n_q_heads + 2 * H) * D}")
    if inv_freq.numel() != D // 2:
        raise ValueError(f"inv_freq must hold head_dim/2 = {D // 2} values")
    _need(block_tables, "block_tables", torch.int32)
    _need(ctx_lens, "ctx_lens", torch.int32)
    if block_tables.dim() != 2 or block_tables.shape[0] != B or not block_tables.is_contiguous():
        raise ValueError("block_tables must be contiguous int32 [B, max_blocks]")
    if ctx_lens.numel() != B:
        raise ValueError("ctx_lens must hold B entries")
    if out is None:
        out = torch.empty((B, n_q_heads, D), dtype=cache_k.dtype, device=cache_k.device)
    need = workspace_bytes(B, n_q_heads, max_ctx, D)
    ws = None
    if need:
        if workspace is not None:
            if workspace.numel() * workspace.element_size() < need:
                raise ValueError(f"workspace holds fewer than the {need} bytes needed")
            ws = workspace
        else:
            ws = get_workspace(need, cache_k.device)
    if ssq is not None:
        _need(ssq, "ssq", torch.float32)
        if ssq.dim() != 2 or ssq.shape[0] != B or not ssq.is_contiguous():
            raise ValueError(f"ssq must be contiguous float32 [{B}, H/16]")
        _lib.call("pdk_decode_attn_rope_rms", qkv_partials.data_ptr(), splits, ssq.data_ptr(),
                  ssq.shape[1], float(eps), inv_freq.data_ptr(), cache_k.data_ptr(),
                  cache_v.data_ptr(), nb, block_tables.data_ptr(), block_tables.shape[1],
                  ctx_lens.data_ptr(), int(max_ctx), B, n_q_heads, H, D, float(scale),
                  ws.data_ptr() if ws is not None else None,
                  ws.numel() * ws.element_size() if ws is not None else 0, out.data_ptr(),
                  int(plan_batch), stream_handle(stream))
        return out
    _lib.call("pdk_decode_attn_rope", qkv_partials.data_ptr(), splits, inv_freq.data_ptr(),
              cache_k.data_ptr(), cache_v.data_ptr(), nb, block_tables.data_ptr(),
              block_tables.shape[1], ctx_lens.data_ptr(), int(max_ctx), B, n_q_heads, H, D,
              float(scale), ws.data_ptr() if ws is not None else None,
              ws.numel() * ws.element_size() if ws is not None else 0, out.data_ptr(),
              int(plan_batch), stream_handle(stream))
    return out


def attn_read_probe(cache_k, cache_v, block_tables, ctx_lens, max_ctx, n_q_heads, out,
                    stream=None):
    """Decode attention's launch with its K/V loads and none of its arithmetic
    (pdk_attn_read_probe): what attention's access pattern costs by itself.
    ``out`` [B, n_q_heads, D] bf16 receives meaningless values."""
    nb, H, D = _check_layer_cache(cache_k, cache_v)
    B = block_tables.shape[0]
    _need(out, "out")
    if tuple(out.shape) != (B, n_q_heads, D):
        raise ValueError(f"out must be [B, n_q_heads, {D}]")
    _lib.call("pdk_attn_read_probe", cache_k.data_ptr(), cache_v.data_ptr(), nb,
              block_tables.data_ptr(), block_tables.shape[1], ctx_lens.data_ptr(), int(max_ctx),
              B, int(n_q_heads), H, D, out.data_ptr(), stream_handle(stream))
    return out


def cache_append(k_new, v_new, cache_k, cache_v, block_tables, ctx_lens, stream=None):
    """Write each stream's new k/v [B, Hkv, D] at slot ctx_lens[b]-1
    (the one-hot injection of kernels/decode_batch.py:81-82)."""
    _need(k_new, "k_new")
    _need(v_new, "v_new")
    nb, H, D = _check_layer_cache(cache_k, cache_v)
    B = k_new.shape[0]
    if tuple(k_new.shape) != (B, H, D) or tuple(v_new.shape) != (B, H, D):
        raise ValueError("k_new/v_new must be [B, Hkv, D]")
    _lib.call("pdk_cache_append", k_new.contiguous().data_ptr(), v_new.contiguous().data_ptr(),
              cache_k.data_ptr(), cache_v.data_ptr(), nb, block_tables.data_ptr(),
              block_tables.shape[1], ctx_lens.data_ptr(), B, H, D, stream_handle(stream))


def greedy_argmax(logits, out=None, stream=None):
    """First-maximum argmax per row of bf16 logits [B, V] -> int32 [B]."""
    _need(logits, "logits")
    if logits.dim() != 2 or logits.stride(1) != 1:
        raise ValueError("logits must be [B, V] with unit column stride")
    B, V = logits.shape
    if out is None:
        out = torch.empty(B, dtype=torch.int32, device=logits.device)
    _lib.call("pdk_greedy_argmax", logits.data_ptr(), B, V, logits.stride(0), out.data_ptr(),
              stream_handle(stream))
    return out
