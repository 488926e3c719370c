"""torch-facing wrappers of the decode step's kernels.

Replace rms_dsl + zipadd_dsl (kernels/dsl_batch.py:22-53), the RoPE rotation
and one-hot cache injection of DecodeLayer.forward (kernels/decode_batch.py:
69-82), swiglu_dsl (kernels/dsl_batch.py:55-71) and the layer's projection
matmuls (kernels/decode_batch.py:73-91). bf16 tensors on the device; fp32
arithmetic inside the kernels.
"""
import torch

from .. import _lib
from .attention import _check_layer_cache
from .handoff import _need, stream_handle


def rmsnorm(x, weight, eps, add=None, out=None, stream=None):
    """out = rmsnorm(x) * weight over the last dim of x [B, H].

    With ``add`` [B, H], x is first replaced in place by bf16(x + add) (the
    residual add), and the norm is taken of that sum."""
    _need(x, "x")
    _need(weight, "weight")
    if x.dim() != 2 or not x.is_contiguous():
        raise ValueError(f"x must be contiguous [B, H], got {tuple(x.shape)}")
    B, H = x.shape
    if weight.numel() != H or not weight.is_contiguous():
        raise ValueError(f"weight must hold H={H} contiguous values")
    if add is not None:
        _need(add, "add")
        if add.shape != x.shape or not add.is_contiguous():
            raise ValueError("add must be contiguous and shaped like x")
    if out is None:
        out = torch.empty_like(x)
    _lib.call("pdk_rmsnorm", x.data_ptr(), add.data_ptr() if add is not None else None,
              weight.data_ptr(), B, H, float(eps), out.data_ptr(), stream_handle(stream))
    return out


def rope_cache_append(qkv, inv_freq, ctx_lens, block_tables, cache_k, cache_v, n_q_heads,
                      q_out=None, stream=None):
    """RoPE at position ctx_lens[b]-1 and the new token's cache write.

    qkv [B, >= (n_q + 2 n_kv) * D] bf16 rows (unit column stride) holding q, k,
    v; inv_freq float32 [D/2]; cache_k [nb, Hkv, 16, D] and cache_v
    [nb, Hkv, D, 16] (one layer). Returns rotated q [B, n_q, D]."""
    _need(qkv, "qkv")
    _need(inv_freq, "inv_freq", torch.float32)
    _need(ctx_lens, "ctx_lens", torch.int32)
    _need(block_tables, "block_tables", torch.int32)
    nb, Hkv, D = _check_layer_cache(cache_k, cache_v)
    if qkv.dim() != 2 or qkv.stride(1) != 1:
        raise ValueError("qkv must be [B, N] with unit column stride")
    B = qkv.shape[0]
    if qkv.shape[1] < (n_q_heads + 2 * Hkv) * D:
        raise ValueError(f"qkv rows hold {qkv.shape[1]} values, need {(n_q_heads + 2 * Hkv) * D}")
    if inv_freq.numel() != D // 2:
        raise ValueError(f"inv_freq must hold head_dim/2 = {D // 2} values")
    if ctx_lens.numel() != B or block_tables.dim() != 2 or block_tables.shape[0] != B \
            or not block_tables.is_contiguous():
        raise ValueError("ctx_lens [B] and contiguous block_tables [B, max_blocks] expected")
    if q_out is None:
        q_out = torch.empty((B, n_q_heads, D), dtype=qkv.dtype, device=qkv.device)
    _lib.call("pdk_rope_cache_append", qkv.data_ptr(), qkv.stride(0), q_out.data_ptr(),
              inv_freq.data_ptr(), ctx_lens.data_ptr(), block_tables.data_ptr(),
              block_tables.shape[1], cache_k.data_ptr(), cache_v.data_ptr(), nb, B, n_q_heads,
              Hkv, D, stream_handle(stream))
    return q_out


def rope_cache_append_partials(partials, inv_freq, ctx_lens, block_tables, cache_k, cache_v,
                               n_q_heads, q_out=None, stream=None, ssq=None, eps=None):
    """rope_cache_append from split-K partial sums of the q|k|v projection.

    partials float32 [splits, B, N] (linear_splitk's output, N = (n_q + 2 n_kv)
    * D), added in split order and rounded to bf16 per element first. With
    ``ssq`` float32 [B, H/16] (the projection's input was the un-normalised
    residual, its weights folded with the norm's gain) each row's sum is
    scaled by r = rsqrt(sum ssq / H + eps) before the rounding."""
    _need(partials, "partials", torch.float32)
    _need(inv_freq, "inv_freq", torch.float32)
    _need(ctx_lens, "ctx_lens", torch.int32)
    _need(block_tables, "block_tables", torch.int32)
    nb, Hkv, D = _check_layer_cache(cache_k, cache_v)
    if partials.dim() != 3 or not partials.is_contiguous():
        raise ValueError("partials must be contiguous [splits, B, N]")
    splits, B, N = partials.shape
    if N != (n_q_heads + 2 * Hkv) * D:
        raise ValueError(f"partials rows hold {N} values, need {(n_q_heads + 2 * Hkv) * D}")
    if inv_freq.numel() != D // 2:
        raise ValueError(f"inv_freq must hold head_dim/2 = {D // 2} values")
    if ctx_lens.numel() != B or block_tables.dim() != 2 or block_tables.shape[0] != B \
            or not block_tables.is_contiguous():
        raise ValueError("ctx_lens [B] and contiguous block_tables [B, max_blocks] expected")
    if q_out is None:
        q_out = torch.empty((B, n_q_heads, D), dtype=cache_k.dtype, device=partials.device)
    if ssq is not None:
        _need(ssq, "ssq", torch.float32)
        if ssq.dim() != 2 or ssq.shape[0] != B or not ssq.is_contiguous():
            raise ValueError(f"ssq must be contiguous float32 [{B}, H/16]")
        _lib.call("pdk_rope_cache_append_partials_rms", partials.data_ptr(), splits, N,
                  ssq.data_ptr(), ssq.shape[1], float(eps), q_out.data_ptr(),
                  inv_freq.data_ptr(), ctx_lens.data_ptr(), block_tables.data_ptr(),
                  block_tables.shape[1], cache_k.data_ptr(), cache_v.data_ptr(), nb, B,
                  n_q_heads, Hkv, D, stream_handle(stream))
        return q_out
    _lib.call("pdk_rope_cache_append_partials", partials.data_ptr(), splits, N, q_out.data_ptr(),
              inv_freq.data_ptr(), ctx_lens.data_ptr(), block_tables.data_ptr(),
              block_tables.shape[1], cache_k.data_ptr(), cache_v.data_ptr(), nb, B, n_q_heads,
              Hkv, D, stream_handle(stream))
    return q_out


def embed_ssq(table, tokens, x=None, ssq=None, stream=None):
    """x = table[tokens] (bf16 [B, H]) and its row_ssq, in one launch; tokens
    int32 or int64 [B] on the device. A token outside [0, vocab) gives a zero
    row (torch's index_select would fault instead)."""
    _need(table, "table")
    if table.dim() != 2 or not table.is_contiguous() or table.shape[1] % 16:
        raise ValueError("table must be contiguous [vocab, H] with H % 16 == 0")
    if tokens.dtype not in (torch.int32, torch.int64) or tokens.dim() != 1 \
            or not tokens.is_cuda or not tokens.is_contiguous():
        raise ValueError("tokens must be a contiguous int32 or int64 [B] device tensor")
    (B,), (V, H) = tokens.shape, table.shape
    if x is None:
        x = torch.empty((B, H), dtype=table.dtype, device=table.device)
    if ssq is None:
        ssq = torch.empty((B, H // 16), dtype=torch.float32, device=table.device)
    if tuple(x.shape) != (B, H) or not x.is_contiguous() or x.dtype != table.dtype:
        raise ValueError(f"x must be contiguous [{B}, {H}] of the table's dtype")
    if ssq.dtype != torch.float32 or not ssq.is_contiguous() or ssq.numel() < B * (H // 16):
        raise ValueError(f"ssq must be contiguous float32 holding {B}x{H // 16}")
    _lib.call("pdk_embed_ssq", table.data_ptr(), V, tokens.data_ptr(), tokens.element_size(), B,
              H, x.data_ptr(), ssq.data_ptr(), stream_handle(stream))
    return x, ssq


def row_ssq(x, ssq=None, stream=None):
    """float32 [B, H/16]: per 16-column tile, the sum of squares of each row
    of the bf16 x [B, H]."""
    _need(x, "x")
    if x.dim() != 2 or not x.is_contiguous() or x.shape[1] % 16:
        raise ValueError("x must be contiguous [B, H] with H % 16 == 0")
    B, H = x.shape
    if ssq is None:
        ssq = torch.empty((B, H // 16), dtype=torch.float32, device=x.device)
    _lib.call("pdk_row_ssq", x.data_ptr(), B, H, ssq.data_ptr(), stream_handle(stream))
    return ssq


def swiglu(gate_up, out=None, stream=None):
    """gate_up [B, 2M] = [g | u] -> silu(g) * u [B, M]."""
    _need(gate_up, "gate_up")
    if gate_up.dim() != 2 or not gate_up.is_contiguous() or gate_up.shape[1] % 2:
        raise ValueError("gate_up must be contiguous [B, 2M]")
    B, M = gate_up.shape[0], gate_up.shape[1] // 2
    if out is None:
        out = torch.empty((B, M), dtype=gate_up.dtype, device=gate_up.device)
    _lib.call("pdk_swiglu", gate_up.data_ptr(), B, M, out.data_ptr(), stream_handle(stream))
    return out


class TiledWeight:
    """A weight [N, K] in the tiled layout of pdk_weight_tile: every 16-row x
    128-column block contiguous, in the order the GEMM kernels read it, and the
    blocks step-major (the first 128 columns of every 16-row tile, then the
    next 128), so the workgroups of a launch read one region of memory at a
    time. ``data`` is the flat bf16 device tensor;
    ``shape`` is the (N, K) of the weight it was made from. The GEMM wrappers
    below take it wherever they take a [N, K] weight, with identical results."""

    __slots__ = ("data", "shape")

    def __init__(self, data, N, K):
        self.data = data
        self.shape = (int(N), int(K))

    def data_ptr(self):
        return self.data.data_ptr()


def tile_weight(w, stream=None):
    """Tiled copy of a contiguous bf16 weight w [N, K] (K % 128 == 0)."""
    _need(w, "w")
    if w.dim() != 2 or not w.is_contiguous():
        raise ValueError("w must be a contiguous [N, K] tensor")
    N, K = w.shape
    n = int(_lib.lib().pdk_weight_tiled_elems(N, K))
    if n == 0:
        raise ValueError(f"cannot tile a [{N}, {K}] weight: K must be a positive multiple of 128")
    data = torch.empty(n, dtype=w.dtype, device=w.device)
    _lib.call("pdk_weight_tile", w.data_ptr(), N, K, data.data_ptr(), stream_handle(stream))
    return TiledWeight(data, N, K)


def act_rows(B):
    """Rows a tiled activation buffer holds for B streams: 16 ceil(B/16)."""
    return (B + 15) // 16 * 16


def act_tile(x):
    """Row-major [B, K] (K % 128 == 0) -> the flat tiled activation layout of
    the _xt entry points (act_rows(B) rows; padding rows zero): the 16 x 128
    block of rows 16t.. and columns 128s.. is contiguous at (t K/128 + s)
    2048, and inside it column 8j + e of row r is at (16 j + r) 8 + e."""
    B, K = x.shape
    if K % 128:
        raise ValueError(f"K={K} must be a multiple of 128")
    Bp = act_rows(B)
    xp = torch.zeros((Bp, K), dtype=x.dtype, device=x.device)
    xp[:B] = x
    # [t, r, s, j, e] -> [t, s, j, r, e]
    return xp.view(Bp // 16, 16, K // 128, 16, 8).permute(0, 2, 3, 1, 4).contiguous().view(-1)


def act_untile(xt, B, K):
    """The inverse of act_tile: rows 0..B-1 of a tiled buffer as [B, K]."""
    Bp = act_rows(B)
    v = xt.view(-1)[:Bp * K].view(Bp // 16, K // 128, 16, 16, 8).permute(0, 3, 1, 2, 4)
    return v.reshape(Bp, K)[:B]


def _check_linear(x, w, rows_per_col=1):
    _need(x, "x")
    if isinstance(w, TiledWeight):
        _need(w.data, "w")
        N, K = w.shape
    else:
        _need(w, "w")
        if w.dim() != 2 or not w.is_contiguous():
            raise ValueError("w must be a contiguous [N, K] tensor or a TiledWeight")
        N, K = w.shape
    if x.dim() != 2 or not x.is_contiguous():
        raise ValueError("x must be a contiguous [B, K] tensor")
    if x.shape[1] != K:
        raise ValueError(f"x has K={x.shape[1]}, w has K={K}")
    if N % rows_per_col:
        raise ValueError("w must hold 2M rows (gate rows, then up rows)")
    return x.shape[0], K, N // rows_per_col


def _entry(name, w):
    return name + "_tiled" if isinstance(w, TiledWeight) else name


def linear(x, w, residual=None, out=None, stream=None):
    """x [B, K] . w[N, K]^T (+ residual [B, N]) -> [B, N], B <= 64 (w in torch
    Linear layout). ``out`` may be ``residual`` (an in-place residual add)."""
    B, K, N = _check_linear(x, w)
    if residual is not None:
        _need(residual, "residual")
        if tuple(residual.shape) != (B, N) or not residual.is_contiguous():
            raise ValueError(f"residual must be contiguous [{B}, {N}]")
    if out is None:
        out = torch.empty((B, N), dtype=x.dtype, device=x.device)
    elif tuple(out.shape) != (B, N) or not out.is_contiguous():
        raise ValueError(f"out must be contiguous [{B}, {N}]")
    _lib.call(_entry("pdk_linear", w), x.data_ptr(), w.data_ptr(), B, K, N,
              residual.data_ptr() if residual is not None else None, out.data_ptr(),
              stream_handle(stream))
    return out


def linear_swiglu(x, w_gate_up, out=None, stream=None):
    """silu(x . wg^T) * (x . wu^T) -> [B, M] for w_gate_up = [wg; wu] [2M, K]."""
    B, K, M = _check_linear(x, w_gate_up, rows_per_col=2)
    if out is None:
        out = torch.empty((B, M), dtype=x.dtype, device=x.device)
    elif tuple(out.shape) != (B, M) or not out.is_contiguous():
        raise ValueError(f"out must be contiguous [{B}, {M}]")
    _lib.call(_entry("pdk_linear_swiglu", w_gate_up), x.data_ptr(), w_gate_up.data_ptr(), B, K, M,
              out.data_ptr(),
              stream_handle(stream))
    return out


def linear_ssq(x, w, residual, ssq, out=None, stream=None):
    """residual + x . w^T -> [B, N] (``out`` may be ``residual``), and ssq
    float32 [B, N/16]: per row and 16-column tile, the sum of squares of the
    bf16 outputs (the raw material of the next RMSNorm)."""
    B, K, N = _check_linear(x, w)
    _need(residual, "residual")
    if tuple(residual.shape) != (B, N) or not residual.is_contiguous():
        raise ValueError(f"residual must be contiguous [{B}, {N}]")
    if N % 16:
        raise ValueError(f"N must be a multiple of 16 (got {N})")
    if ssq.dtype != torch.float32 or not ssq.is_cuda or not ssq.is_contiguous() \
            or ssq.numel() < (N // 16) * B:
        raise ValueError(f"ssq must be contiguous float32 holding {N // 16}x{B}")
    if out is None:
        out = torch.empty((B, N), dtype=x.dtype, device=x.device)
    elif tuple(out.shape) != (B, N) or not out.is_contiguous():
        raise ValueError(f"out must be contiguous [{B}, {N}]")
    _lib.call(_entry("pdk_linear_ssq", w), x.data_ptr(), w.data_ptr(), B, K, N,
              residual.data_ptr(), out.data_ptr(), ssq.data_ptr(), stream_handle(stream))
    return out


def fold_norm(w, g):
    """w [N, K] with the RMSNorm gain g [K] folded into its columns:
    bf16(w * g), the weight linear_swiglu_rms takes."""
    _need(w, "w")
    _need(g, "g")
    if w.dim() != 2 or g.shape != (w.shape[1],):
        raise ValueError(f"g must be [{w.shape[1]}] for w {tuple(w.shape)}")
    return (w.float() * g.float()[None, :]).to(w.dtype).contiguous()


def linear_swiglu_rms(x, w_gate_up_folded, ssq, eps, out=None, stream=None):
    """silu(r x . wg'^T) * (r x . wu'^T) -> [B, M], r_b = rsqrt(sum_t ssq[b, t]
    / K + eps): the gate|up of rmsnorm(x) * g for weights folded with g
    (fold_norm), ssq from the linear_ssq that produced x."""
    B, K, M = _check_linear(x, w_gate_up_folded, rows_per_col=2)
    if ssq.dtype != torch.float32 or not ssq.is_cuda or not ssq.is_contiguous() \
            or ssq.numel() < (K // 16) * B:
        raise ValueError(f"ssq must be contiguous float32 holding {K // 16}x{B}")
    if out is None:
        out = torch.empty((B, M), dtype=x.dtype, device=x.device)
    elif tuple(out.shape) != (B, M) or not out.is_contiguous():
        raise ValueError(f"out must be contiguous [{B}, {M}]")
    _lib.call(_entry("pdk_linear_swiglu_rms", w_gate_up_folded), x.data_ptr(),
              w_gate_up_folded.data_ptr(), B, K, M, ssq.data_ptr(), K // 16, float(eps),
              out.data_ptr(), stream_handle(stream))
    return out


def linear_splitk_rms(x, w_folded, splits, ssq, eps, partials=None, stream=None):
    """linear_splitk of rmsnorm(x) * g for weights folded with g (fold_norm):
    each row's partials scaled by r from ssq [B, K/16]."""
    B, K, N = _check_linear(x, w_folded)
    if ssq.dtype != torch.float32 or ssq.numel() < (K // 16) * B or not ssq.is_contiguous():
        raise ValueError(f"ssq must be contiguous float32 holding {B}x{K // 16}")
    if partials is None:
        partials = torch.empty((splits, B, N), dtype=torch.float32, device=x.device)
    _lib.call(_entry("pdk_linear_splitk_rms", w_folded), x.data_ptr(), w_folded.data_ptr(), B, K,
              N, int(splits), ssq.data_ptr(), K // 16, float(eps), partials.data_ptr(),
              stream_handle(stream))
    return partials


def linear_splitk_final(x, w, splits, residual, ssq, counters, partials=None, stream=None):
    """residual += x . w^T in place (bf16(residual + sum of split-K partials in
    split order), added by the last split of each column group) and ssq
    float32 [B, N/16] of the result; counters: int32 device zeros (>= N/16),
    left zero."""
    B, K, N = _check_linear(x, w)
    _need(residual, "residual")
    if tuple(residual.shape) != (B, N) or not residual.is_contiguous():
        raise ValueError(f"residual must be contiguous [{B}, {N}]")
    if ssq.dtype != torch.float32 or ssq.numel() < (N // 16) * B or not ssq.is_contiguous():
        raise ValueError(f"ssq must be contiguous float32 holding {N // 16}x{B}")
    if counters.dtype != torch.int32 or counters.numel() < N // 16:
        raise ValueError(f"counters must be int32 holding >= {N // 16} zeros")
    if partials is None:
        partials = torch.empty((splits, B, N), dtype=torch.float32, device=x.device)
    _lib.call(_entry("pdk_linear_splitk_final", w), x.data_ptr(), w.data_ptr(), B, K, N,
              int(splits), partials.data_ptr(), residual.data_ptr(), ssq.data_ptr(),
              counters.data_ptr(), stream_handle(stream))
    return residual


def linear_argmax_rms(x, w_folded, ssq, eps, keys, tokens=None, logits=None, stream=None):
    """linear_argmax of rmsnorm(x) * g for weights folded with g (fold_norm):
    each row's logits scaled by r from ssq [B, K/16] before rounding."""
    B, K, N = _check_linear(x, w_folded)
    if ssq.dtype != torch.float32 or ssq.numel() < (K // 16) * B or not ssq.is_contiguous():
        raise ValueError(f"ssq must be contiguous float32 holding {K // 16}x{B}")
    if tokens is None:
        tokens = torch.empty(B, dtype=torch.int32, device=x.device)
    _lib.call(_entry("pdk_linear_argmax_rms", w_folded), x.data_ptr(), w_folded.data_ptr(), B, K,
              N, ssq.data_ptr(), K // 16, float(eps),
              logits.data_ptr() if logits is not None else None, keys.data_ptr(),
              tokens.data_ptr(), stream_handle(stream))
    return tokens


def linear_argmax(x, w, keys, tokens=None, logits=None, stream=None):
    """Greedy tokens of x . w^T (the lm_head): the first-maximum argmax of each
    row of the bf16 logits, computed in the GEMM's epilogue. ``keys`` is an
    int64 [>= B] device scratch holding zeros (left zero); ``logits`` [B, N]
    receives the logits when given. Returns int32 [B] tokens."""
    B, K, N = _check_linear(x, w)
    if not isinstance(keys, torch.Tensor) or not keys.is_cuda or keys.dtype != torch.int64 \
            or keys.numel() < B or not keys.is_contiguous():
        raise ValueError(f"keys must be a contiguous CUDA int64 tensor of >= {B} zeros")
    if tokens is None:
        tokens = torch.empty(B, dtype=torch.int32, device=x.device)
    if logits is not None and (tuple(logits.shape) != (B, N) or not logits.is_contiguous()):
        raise ValueError(f"logits must be contiguous [{B}, {N}]")
    _lib.call(_entry("pdk_linear_argmax", w), x.data_ptr(), w.data_ptr(), B, K, N,
              logits.data_ptr() if logits is not None else None, keys.data_ptr(),
              tokens.data_ptr(), stream_handle(stream))
    return tokens


def linear_splitk(x, w, splits, partials=None, stream=None):
    """x . w^T split over K into fp32 partial sums [splits, B, N] (summed
    later, e.g. by rmsnorm_partials)."""
    B, K, N = _check_linear(x, w)
    if partials is None:
        partials = torch.empty((splits, B, N), dtype=torch.float32, device=x.device)
    elif partials.dtype != torch.float32 or partials.numel() < splits * B * N or \
            not partials.is_contiguous():
        raise ValueError(f"partials must be contiguous float32 holding {splits}x{B}x{N}")
    _lib.call(_entry("pdk_linear_splitk", w), x.data_ptr(), w.data_ptr(), B, K, N, int(splits),
              partials.data_ptr(), stream_handle(stream))
    return partials


def rmsnorm_partials(x, partials, splits, weight, eps, out=None, stream=None):
    """x <- bf16(x + sum of partials[:splits]) in place, then rmsnorm(x) * weight."""
    _need(x, "x")
    _need(weight, "weight")
    if x.dim() != 2 or not x.is_contiguous():
        raise ValueError("x must be contiguous [B, H]")
    B, H = x.shape
    if partials.dtype != torch.float32 or partials.numel() < splits * B * H:
        raise ValueError(f"partials must be float32 holding {splits}x{B}x{H}")
    if out is None:
        out = torch.empty_like(x)
    _lib.call("pdk_rmsnorm_partials", x.data_ptr(), partials.data_ptr(), int(splits),
              weight.data_ptr(), B, H, float(eps), out.data_ptr(), stream_handle(stream))
    return out
