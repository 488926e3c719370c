"""numpy restatement of the reference's full decode step -- TEST INFRASTRUCTURE.

Only the tests, the smoke check and the CPU-baseline leg of the benchmark use
this module, and only as the oracle results are compared with: no product path imports it.

Follows cpu_layer (kernels/decode_batch.py:124-162) for one layer of B streams
at their own positions, ModelConfig.inv_freq (engines/model.py:32-50) for the
llama3-scaled RoPE frequencies, rope/rmsnorm (engines/model.py:53-65) and
greedy_tokens (engines/decode_batch.py:162-171) for the head. All arithmetic is
float32 (float64 for inv_freq before its float32 cast, as the reference does).

Layout: weights are [in, out] (the transpose of torch Linear weights, which
cpu_layer applies as ``h @ w.T``), with q|k|v and gate|up concatenated along
``out``; per-stream dense caches are K [B, NKV, S, HD] and V [B, NKV, S, HD]
(token-major for both; cpu_layer keeps K as [.., HD, S], the same values).
"""
import math

import numpy as np


def inv_freq(head_dim, theta, rope_scaling=None):
    """float32 [head_dim/2]: theta^(-2i/d) in float64, then the llama3 band
    scaling (engines/model.py:32-50) when ``rope_scaling`` = (factor,
    low_freq_factor, high_freq_factor, original_max_position_embeddings)."""
    inv = 1.0 / (theta ** (np.arange(0, head_dim, 2, dtype=np.float64) / head_dim))
    if rope_scaling:
        factor, lo, hi, orig = rope_scaling
        low_wl, high_wl = orig / lo, orig / hi
        wl = 2 * math.pi / inv
        smooth = (orig / wl - lo) / (hi - lo)
        inv = np.where(wl > low_wl, inv / factor,
                       np.where(wl < high_wl, inv, (1 - smooth) * inv / factor + smooth * inv))
    return inv.astype(np.float32)


def rmsnorm(x, w, eps):
    """Rows of x [.., H]: x / sqrt(mean(x^2) + eps) * w (kernels/decode_batch.py:129)."""
    x = np.asarray(x, np.float32)
    return x * (1.0 / np.sqrt((x * x).mean(-1, keepdims=True) + eps)) * w


def rope(t, positions, inv):
    """Rotate-half RoPE of t [B, nh, HD] at positions[b] (kernels/decode_batch.py:132-141):
    the angle pos*inv[i] in float32, (a, b) -> (a cos - b sin, b cos + a sin)
    for the two halves of each head."""
    t = np.array(t, np.float32)
    half = t.shape[-1] // 2
    for b, p in enumerate(positions):
        ang = np.float32(p) * inv
        cs, sn = np.cos(ang), np.sin(ang)
        a, c = t[b, :, :half].copy(), t[b, :, half:].copy()
        t[b, :, :half] = a * cs - c * sn
        t[b, :, half:] = c * cs + a * sn
    return t


def swiglu(gu):
    """[.., 2M] = [g | u] -> silu(g) * u (kernels/decode_batch.py:159-160)."""
    M = gu.shape[-1] // 2
    g, u = gu[..., :M], gu[..., M:]
    with np.errstate(over="ignore"):             # exp(-g) -> inf gives silu(g) = -0
        return g / (1 + np.exp(-g)) * u


def attention(q, K, V, positions):
    """q [B, NH, HD] after RoPE; K/V [B, NKV, S, HD] with the new token already
    at positions[b]. Scores q.k / sqrt(HD), slots after pos masked to -1e4,
    max-subtracted softmax, p.V (kernels/decode_batch.py:151-156)."""
    B, NH, HD = q.shape
    NKV = K.shape[1]
    G = NH // NKV
    sc = np.einsum("bkgh,bksh->bkgs", q.reshape(B, NKV, G, HD), K) / math.sqrt(HD)
    for b, p in enumerate(positions):
        sc[b, :, :, p + 1:] = -1e4
    sc = sc - sc.max(-1, keepdims=True)
    pr = np.exp(sc)
    pr /= pr.sum(-1, keepdims=True)
    return np.einsum("bkgs,bksh->bkgh", pr, V).reshape(B, NH, HD)


def decode_layer(x, lw, K, V, inv, positions, n_heads, n_kv_heads, eps):
    """One layer for B streams (cpu_layer, kernels/decode_batch.py:124-162).

    x float32 [B, H]; lw = (norm1, wqkv, wo, norm2, wgu, wd) float32 in [in, out]
    layout; K, V float32 [B, NKV, S, HD], updated in place at positions[b].
    Returns the layer's output hidden state [B, H]."""
    norm1, wqkv, wo, norm2, wgu, wd = lw
    B = x.shape[0]
    HD = K.shape[-1]
    h = rmsnorm(x, norm1, eps)
    qkv = h @ wqkv
    nq = n_heads * HD
    nk = n_kv_heads * HD
    q = rope(qkv[:, :nq].reshape(B, n_heads, HD), positions, inv)
    k = rope(qkv[:, nq:nq + nk].reshape(B, n_kv_heads, HD), positions, inv)
    v = qkv[:, nq + nk:nq + 2 * nk].reshape(B, n_kv_heads, HD)
    for b, p in enumerate(positions):
        K[b, :, p, :] = k[b]
        V[b, :, p, :] = v[b]
    ao = attention(q, K, V, positions).reshape(B, nq)
    x2 = ao @ wo + x
    h2 = rmsnorm(x2, norm2, eps)
    return swiglu(h2 @ wgu) @ wd + x2


def decode_step(tokens, weights, Ks, Vs, positions, cfg):
    """One greedy step: embed -> layers -> final norm -> lm_head -> first-max argmax
    (greedy_tokens, engines/decode_batch.py:162-171; numpy's argmax returns the
    first maximum, as torch.argmax does).

    weights: dict of float32 arrays embed [V, H], layers [(norm1, wqkv, wo,
    norm2, wgu, wd)], norm_f [H], lm_head [H, V]; Ks/Vs per layer [B, NKV, S, HD]
    (updated). cfg: object with n_heads, n_kv_heads, eps, inv (float32 [HD/2]).
    Returns (next tokens int64 [B], hidden before the final norm [B, H],
    logits [B, V])."""
    x = weights["embed"][np.asarray(tokens)]
    for li, lw in enumerate(weights["layers"]):
        x = decode_layer(x, lw, Ks[li], Vs[li], cfg.inv, positions, cfg.n_heads, cfg.n_kv_heads,
                         cfg.eps)
    logits = rmsnorm(x, weights["norm_f"], cfg.eps) @ weights["lm_head"]
    return np.argmax(logits, axis=-1), x, logits


def rel_l2(got, want):
    """||got - want|| / ||want|| (the reference's hidden-state check,
    kernels/decode_batch.py:290-294, which passes below 0.08)."""
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    return float(np.linalg.norm(got - want) / np.linalg.norm(want))
