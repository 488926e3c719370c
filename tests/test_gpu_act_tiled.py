"""The decode step's tiled-activation entry points (the *_xt family).

Each *_xt entry point is its row-major namesake with the bf16 activations (x,
the residual, y, attention's output) in the tiled layout of act_tile. The
arithmetic is the same, summed in the same order, so after act_untile every
output must equal the row-major entry point's bit for bit. Inputs' padding
rows (past B in the last 16-row tile) hold NaN: the kernels must never read
them.
"""
import math

import numpy as np
import pytest
import torch

from oracle import decode as od
from rngd_pd_amd import _lib
from tests._util import rand_bf16, to_dev

pytestmark = pytest.mark.gpu

BF16 = torch.bfloat16
LLAMA3 = (8.0, 1.0, 4.0, 8192)


def _tiled_in(x):
    """act_tile(x) with NaN in the padding rows."""
    from rngd_pd_amd import kernels as K_
    B, K = x.shape
    rows = K_.act_rows(B)
    full = torch.full((rows, K), float("nan"), dtype=x.dtype, device=x.device)
    full[:B] = x
    t = K_.act_tile(full)
    return t


def _eq(a, b):
    return torch.equal(a.contiguous().view(torch.int16), b.contiguous().view(torch.int16))


@pytest.mark.parametrize("B,K,N", [(1, 128, 128), (4, 4096, 4096), (16, 4096, 4096),
                                   (17, 512, 1024), (33, 256, 384), (64, 128, 256)])
def test_xt_ssq_and_splitk_equal_row_major(cuda, B, K, N):
    from rngd_pd_amd import kernels as K_
    rng = np.random.default_rng(B * 7 + K + N)
    x, w, r = rand_bf16(rng, (B, K)), rand_bf16(rng, (N, K), 0.05), rand_bf16(rng, (B, N), 4.0)
    xd, rd = to_dev(x), to_dev(r)
    wt = K_.tile_weight(to_dev(w))
    print(f"xt ssq/splitk B={B} K={K} N={N}", flush=True)
    # O projection: y = r + x . w^T, with the sums of squares.
    y_ref = rd.clone()
    ssq_ref = torch.zeros((B, N // 16), dtype=torch.float32, device=cuda)
    _lib.call("pdk_linear_ssq_tiled", xd.data_ptr(), wt.data_ptr(), B, K, N, y_ref.data_ptr(),
              y_ref.data_ptr(), ssq_ref.data_ptr(), 0)
    y_t = _tiled_in(rd)
    ssq = torch.full((B, N // 16), float("nan"), dtype=torch.float32, device=cuda)
    _lib.call("pdk_linear_ssq_xt", _tiled_in(xd).data_ptr(), wt.data_ptr(), B, K, N,
              y_t.data_ptr(), y_t.data_ptr(), ssq.data_ptr(), 0)
    # q|k|v: fp32 split partials scaled by the row's r.
    ssq_in = torch.from_numpy(rng.random((B, K // 16)).astype(np.float32) + 0.5).to(cuda)
    splits = 2 if K >= 256 else 1
    p_ref = torch.zeros((splits, B, N), dtype=torch.float32, device=cuda)
    p_xt = torch.full((splits, B, N), float("nan"), dtype=torch.float32, device=cuda)
    _lib.call("pdk_linear_splitk_rms_tiled", xd.data_ptr(), wt.data_ptr(), B, K, N, splits,
              ssq_in.data_ptr(), K // 16, 1e-5, p_ref.data_ptr(), 0)
    _lib.call("pdk_linear_splitk_rms_xt", _tiled_in(xd).data_ptr(), wt.data_ptr(), B, K, N,
              splits, ssq_in.data_ptr(), K // 16, 1e-5, p_xt.data_ptr(), 0)
    torch.cuda.synchronize()
    assert _eq(K_.act_untile(y_t, B, N), y_ref)
    assert torch.equal(ssq, ssq_ref)
    assert torch.equal(p_xt, p_ref)


@pytest.mark.parametrize("B,K,M", [(16, 4096, 14336), (4, 4096, 14336), (3, 256, 128),
                                   (20, 512, 256), (40, 128, 512)])
def test_xt_swiglu_equals_row_major(cuda, B, K, M):
    from rngd_pd_amd import kernels as K_
    rng = np.random.default_rng(B + K + M)
    x, w = rand_bf16(rng, (B, K)), rand_bf16(rng, (2 * M, K), 0.05)
    xd = to_dev(x)
    wt = K_.tile_weight(to_dev(w))
    ssq = torch.from_numpy(rng.random((B, K // 16)).astype(np.float32) + 0.5).to(cuda)
    print(f"xt swiglu B={B} K={K} M={M}", flush=True)
    y_ref = torch.empty((B, M), dtype=BF16, device=cuda)
    _lib.call("pdk_linear_swiglu_rms_tiled", xd.data_ptr(), wt.data_ptr(), B, K, M,
              ssq.data_ptr(), K // 16, 1e-5, y_ref.data_ptr(), 0)
    y_t = torch.full((K_.act_rows(B) * M,), float("nan"), dtype=BF16, device=cuda)
    _lib.call("pdk_linear_swiglu_rms_xt", _tiled_in(xd).data_ptr(), wt.data_ptr(), B, K, M,
              ssq.data_ptr(), K // 16, 1e-5, y_t.data_ptr(), 0)
    torch.cuda.synchronize()
    assert _eq(K_.act_untile(y_t, B, M), y_ref)


@pytest.mark.parametrize("B,K,N,splits", [(16, 14336, 4096, 2), (4, 14336, 4096, 2),
                                          (33, 512, 1024, 2), (1, 128, 128, 1)])
def test_xt_splitk_final_equals_row_major(cuda, B, K, N, splits):
    from rngd_pd_amd import kernels as K_
    rng = np.random.default_rng(B * 3 + K + N)
    x, w, r = rand_bf16(rng, (B, K)), rand_bf16(rng, (N, K), 0.05), rand_bf16(rng, (B, N), 4.0)
    xd, rd = to_dev(x), to_dev(r)
    wt = K_.tile_weight(to_dev(w))
    counters = torch.zeros(N // 16, dtype=torch.int32, device=cuda)
    part = torch.empty((splits, B, N), dtype=torch.float32, device=cuda)
    print(f"xt splitk_final B={B} K={K} N={N} splits={splits}", flush=True)
    for call in range(2):                                     # counters back at zero each call
        y_ref = rd.clone()
        ssq_ref = torch.zeros((B, N // 16), dtype=torch.float32, device=cuda)
        _lib.call("pdk_linear_splitk_final_tiled", xd.data_ptr(), wt.data_ptr(), B, K, N, splits,
                  part.data_ptr(), y_ref.data_ptr(), ssq_ref.data_ptr(), counters.data_ptr(), 0)
        y_t = _tiled_in(rd)
        ssq = torch.full((B, N // 16), float("nan"), dtype=torch.float32, device=cuda)
        _lib.call("pdk_linear_splitk_final_xt", _tiled_in(xd).data_ptr(), wt.data_ptr(), B, K,
                  N, splits, part.data_ptr(), y_t.data_ptr(), ssq.data_ptr(),
                  counters.data_ptr(), 0)
        torch.cuda.synchronize()
        assert _eq(K_.act_untile(y_t, B, N), y_ref), call
        assert torch.equal(ssq, ssq_ref), call
        assert int(counters.abs().sum()) == 0, call


@pytest.mark.parametrize("B,K,N", [(16, 4096, 128256), (4, 4096, 128256), (3, 256, 1000),
                                   (20, 128, 4096)])
def test_xt_argmax_equals_row_major(cuda, B, K, N):
    from rngd_pd_amd import kernels as K_
    rng = np.random.default_rng(B + 2 * K + N)
    x, w = rand_bf16(rng, (B, K)), rand_bf16(rng, (N, K), 0.05)
    xd = to_dev(x)
    wt = K_.tile_weight(to_dev(w))
    ssq = torch.from_numpy(rng.random((B, K // 16)).astype(np.float32) + 0.5).to(cuda)
    print(f"xt argmax B={B} K={K} N={N}", flush=True)
    outs = []
    for name, xin in (("pdk_linear_argmax_rms_tiled", xd), ("pdk_linear_argmax_rms_xt",
                                                             _tiled_in(xd))):
        logits = torch.empty((B, N), dtype=BF16, device=cuda)
        keys = torch.zeros(B, dtype=torch.int64, device=cuda)
        tok = torch.full((B,), -1, dtype=torch.int32, device=cuda)
        _lib.call(name, xin.data_ptr(), wt.data_ptr(), B, K, N, ssq.data_ptr(), K // 16, 1e-5,
                  logits.data_ptr(), keys.data_ptr(), tok.data_ptr(), 0)
        outs.append((logits, tok))
    torch.cuda.synchronize()
    assert _eq(outs[1][0], outs[0][0])                    # logits stay row-major
    assert torch.equal(outs[1][1], outs[0][1])


def test_xt_embed_equals_row_major(cuda):
    from rngd_pd_amd import kernels as K_
    rng = np.random.default_rng(9)
    V, H = 1000, 4096
    table = to_dev(rand_bf16(rng, (V, H), 2.0))
    for B in (1, 16, 21):
        ids = rng.integers(0, V, B)
        ids[0] = -1 if B > 1 else ids[0]
        tok = torch.from_numpy(ids).to(cuda)
        print(f"xt embed B={B}", flush=True)
        x_ref, ssq_ref = K_.embed_ssq(table, tok)
        xt = torch.full((K_.act_rows(B) * H,), float("nan"), dtype=BF16, device=cuda)
        ssq = torch.empty((B, H // 16), dtype=torch.float32, device=cuda)
        _lib.call("pdk_embed_ssq_xt", table.data_ptr(), V, tok.data_ptr(), 8, B, H,
                  xt.data_ptr(), ssq.data_ptr(), 0)
        torch.cuda.synchronize()
        assert _eq(K_.act_untile(xt, B, H), x_ref)
        assert torch.equal(ssq, ssq_ref)


@pytest.mark.parametrize("B,splits,ctx", [(16, 2, 512), (4, 2, 600), (1, 1, 1500),
                                          (5, 2, 2000), (17, 2, 300)])
def test_xt_fused_attention_equals_row_major(cuda, B, splits, ctx):
    """Attention's output tiled, on one context split and on several (the merge
    launch writes it then); the cache writes are the same either way."""
    from rngd_pd_amd import kernels as K_
    D, NH, NKV = 128, 32, 8
    rng = np.random.default_rng(B * 11 + ctx)
    ctxs = [max(1, ctx - 37 * i) for i in range(B)]
    max_blocks = (max(ctxs) + 15) // 16
    nb = B * max_blocks + 3
    tables = rng.permutation(nb)[:B * max_blocks].astype(np.int32).reshape(B, max_blocks)
    N = (NH + 2 * NKV) * D
    part = torch.from_numpy((rng.standard_normal((splits, B, N)) * 2).astype(np.float32)).to(cuda)
    ck0, cv0 = rand_bf16(rng, (nb, NKV, 16, D)), rand_bf16(rng, (nb, NKV, D, 16))
    inv = torch.from_numpy(od.inv_freq(D, 500000.0, LLAMA3)).to(cuda)
    ctx_t = torch.tensor(ctxs, dtype=torch.int32, device=cuda)
    tab = torch.from_numpy(tables).to(cuda)
    scale = 1.0 / math.sqrt(D)
    print(f"xt fused attention B={B} splits={splits} ctx={ctxs[:4]}", flush=True)
    wsb = K_.workspace_bytes(B, NH, max(ctxs), D)
    ws = torch.zeros(max(wsb, 4) // 4, dtype=torch.float32, device=cuda)
    ck_a, cv_a = to_dev(ck0), to_dev(cv0)
    out_a = K_.decode_attention_rope(part, inv, ck_a, cv_a, tab, ctx_t, max(ctxs), NH,
                                     scale=scale)
    ck_b, cv_b = to_dev(ck0), to_dev(cv0)
    out_t = torch.full((K_.act_rows(B) * NH * D,), float("nan"), dtype=BF16, device=cuda)
    _lib.call("pdk_decode_attn_rope_xt", part.data_ptr(), splits, inv.data_ptr(),
              ck_b.data_ptr(), cv_b.data_ptr(), nb, tab.data_ptr(), max_blocks,
              ctx_t.data_ptr(), max(ctxs), B, NH, NKV, D, scale,
              ws.data_ptr(), wsb, out_t.data_ptr(), B, 0)
    torch.cuda.synchronize()
    assert _eq(K_.act_untile(out_t, B, NH * D), out_a.view(B, NH * D))
    assert _eq(ck_b, ck_a) and _eq(cv_b, cv_a)
