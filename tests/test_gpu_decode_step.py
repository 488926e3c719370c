"""The decode step on the GPU against the oracle's restatement of cpu_layer.

Kernel by kernel (RMSNorm with the residual add, RoPE with the cache write,
SwiGLU), then whole steps of the Llama decoder over a paged cache holding
random prefilled KV. The whole-step bar is the reference's own
(kernels/decode_batch.py:285-294: hidden-state rel L2 below 0.08 against the
fp32 CPU layer); the test also holds a tighter bound that bf16 activations
meet, and greedy tokens must equal the oracle's wherever the oracle's top-two
logit margin exceeds the measured logit error.
"""
import math

import numpy as np
import pytest
import torch

from oracle import attention as oatt
from oracle import decode as od
from tests._util import rand_bf16, to_dev, to_host

pytestmark = pytest.mark.gpu

BF16 = torch.bfloat16
HALF_ULP = 2.0 ** -8            # bf16 round-to-nearest: relative error at most 2^-8
LLAMA3 = (8.0, 1.0, 4.0, 8192)
REL_REFERENCE_BAR = 0.08        # kernels/decode_batch.py:294
REL_TIGHT = 0.02


def _f32(u16):
    return (np.asarray(u16).astype(np.uint32) << 16).view(np.float32)


def _bf16_bits_rne(x_f32):
    t = torch.from_numpy(np.ascontiguousarray(x_f32, np.float32)).to(BF16)
    return t.view(torch.int16).numpy().view(np.uint16)


# ---- kernels -----------------------------------------------------------------

@pytest.mark.parametrize("B,H", [(1, 4096), (5, 512), (3, 8192), (2, 8)])
def test_rmsnorm_and_residual_add(cuda, B, H):
    from rngd_pd_amd import kernels as K
    rng = np.random.default_rng(B * 7 + H)
    x, add = rand_bf16(rng, (B, H), 2.0), rand_bf16(rng, (B, H), 2.0)
    w = rand_bf16(rng, (H,))
    xd, addd, wd = to_dev(x), to_dev(add), to_dev(w)
    print(f"rmsnorm B={B} H={H}", flush=True)
    out = K.rmsnorm(xd, wd, 1e-5)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(to_host(xd), x)                 # no add: x untouched
    np.testing.assert_allclose(_f32(to_host(out)), od.rmsnorm(_f32(x), _f32(w), 1e-5),
                               rtol=HALF_ULP, atol=1e-6)
    out = K.rmsnorm(xd, wd, 1e-5, add=addd)
    torch.cuda.synchronize()
    summed = _bf16_bits_rne(_f32(x) + _f32(add))                  # one fp32 add, then RNE
    np.testing.assert_array_equal(to_host(xd), summed)
    np.testing.assert_allclose(_f32(to_host(out)), od.rmsnorm(_f32(summed), _f32(w), 1e-5),
                               rtol=HALF_ULP, atol=1e-6)


@pytest.mark.parametrize("D", [128, 64])
def test_rope_and_cache_write(cuda, D):
    from rngd_pd_amd import kernels as K
    NH, NKV = 8, 2
    positions = [0, 15, 16, 33, 4095, 99999]
    B = len(positions)
    rng = np.random.default_rng(D)
    max_blocks = max(positions) // 16 + 1
    nb = 2 * B + 1
    tables = np.zeros((B, max_blocks), np.int32)                  # unused entries name block 0
    own = rng.permutation(np.arange(1, nb))[:B]                   # one distinct block per stream
    for b, p in enumerate(positions):
        tables[b, p // 16] = own[b]
    N = (NH + 2 * NKV) * D
    qkv_full = rand_bf16(rng, (B, N + 24))                        # row stride wider than a row
    ck0, cv0 = rand_bf16(rng, (nb, NKV, 16, D)), rand_bf16(rng, (nb, NKV, D, 16))
    ck, cv = to_dev(ck0), to_dev(cv0)
    inv = od.inv_freq(D, 500000.0, LLAMA3)
    print(f"rope_cache_append D={D} positions={positions}", flush=True)
    q = K.rope_cache_append(to_dev(qkv_full)[:, :N], torch.from_numpy(inv).to(cuda),
                            torch.tensor([p + 1 for p in positions], dtype=torch.int32,
                                         device=cuda),
                            torch.from_numpy(tables).to(cuda), ck, cv, NH)
    torch.cuda.synchronize()
    qkv = _f32(qkv_full[:, :N])
    want_q = od.rope(qkv[:, :NH * D].reshape(B, NH, D), positions, inv)
    np.testing.assert_allclose(_f32(to_host(q)), want_q, rtol=HALF_ULP, atol=1e-5)
    want_k = od.rope(qkv[:, NH * D:(NH + NKV) * D].reshape(B, NKV, D), positions, inv)
    v_bits = qkv_full[:, (NH + NKV) * D:N].reshape(B, NKV, D)
    got_k, got_v = to_host(ck), to_host(cv)
    rows_got, rows_0 = oatt.k_block_rows(got_k), oatt.k_block_rows(ck0)
    expect_k, expect_v = rows_0.copy(), cv0.copy()
    for b, p in enumerate(positions):
        blk, slot = own[b], p % 16
        np.testing.assert_allclose(_f32(rows_got[blk, :, slot, :]), want_k[b], rtol=HALF_ULP,
                                   atol=1e-5)
        expect_k[blk, :, slot, :] = rows_got[blk, :, slot, :]
        expect_v[blk, :, :, slot] = v_bits[b]                      # v is copied bit for bit
    np.testing.assert_array_equal(rows_got, expect_k)              # nothing else changed
    np.testing.assert_array_equal(got_v, expect_v)


@pytest.mark.parametrize("splits", [1, 2, 4])
def test_rope_from_partials_equals_rounded_sum(cuda, splits):
    """Split-K partials of the q|k|v projection: the kernel adds them in split
    order in fp32, rounds once to bf16, then does exactly what the bf16-row
    kernel does on that row (bit-for-bit equal q, K and V cache contents)."""
    from rngd_pd_amd import kernels as K
    NH, NKV, D = 8, 2, 128
    positions = [0, 17, 511, 4000]
    B = len(positions)
    rng = np.random.default_rng(100 + splits)
    max_blocks = max(positions) // 16 + 1
    nb = 2 * B + 1
    tables = np.zeros((B, max_blocks), np.int32)
    own = rng.permutation(np.arange(1, nb))[:B]
    for b, p in enumerate(positions):
        tables[b, p // 16] = own[b]
    N = (NH + 2 * NKV) * D
    part = (rng.standard_normal((splits, B, N)) * 3).astype(np.float32)
    total = part[0].copy()
    for s in range(1, splits):
        total = total + part[s]                                    # float32, split order
    rows = _bf16_bits_rne(total)
    ck0, cv0 = rand_bf16(rng, (nb, NKV, 16, D)), rand_bf16(rng, (nb, NKV, D, 16))
    inv = torch.from_numpy(od.inv_freq(D, 500000.0, LLAMA3)).to(cuda)
    ctx = torch.tensor([p + 1 for p in positions], dtype=torch.int32, device=cuda)
    tab = torch.from_numpy(tables).to(cuda)
    print(f"rope_cache_append_partials splits={splits} positions={positions}", flush=True)
    ck_a, cv_a = to_dev(ck0), to_dev(cv0)
    q_a = K.rope_cache_append_partials(torch.from_numpy(part).to(cuda), inv, ctx, tab, ck_a, cv_a,
                                       NH)
    ck_b, cv_b = to_dev(ck0), to_dev(cv0)
    q_b = K.rope_cache_append(to_dev(rows), inv, ctx, tab, ck_b, cv_b, NH)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(to_host(q_a), to_host(q_b))
    np.testing.assert_array_equal(to_host(ck_a), to_host(ck_b))
    np.testing.assert_array_equal(to_host(cv_a), to_host(cv_b))
    # and the V slots hold the rounded sums themselves
    got_v = to_host(cv_a)
    for b, p in enumerate(positions):
        np.testing.assert_array_equal(got_v[own[b], :, :, p % 16],
                                      rows[b, (NH + NKV) * D:].reshape(NKV, D))


@pytest.mark.parametrize("B,splits,NH,NKV", [(16, 2, 32, 8), (4, 2, 32, 8), (1, 1, 32, 8),
                                             (5, 4, 32, 8), (4, 2, 8, 8), (3, 1, 16, 8),
                                             (6, 2, 64, 8), (2, 4, 32, 2), (16, 1, 16, 1),
                                             # units in a partial group of 8, query heads
                                             # shared by 2 or 4 workgroups
                                             (5, 2, 12, 3), (7, 1, 6, 3)])
def test_fused_rope_attention_equals_two_calls(cuda, B, splits, NH, NKV):
    """pdk_decode_attn_rope against pdk_rope_cache_append_partials followed by
    pdk_decode_attn on copies of the same cache: bit-identical outputs and
    cache contents, over context lengths that put the new token at a block's
    first, last and middle slot, past one workgroup's 512 tokens, in the
    context splits of small batches, and in a block whose id is invalid (no
    cache write on either path); GQA groups of 1 to 16 query heads."""
    from rngd_pd_amd import kernels as K
    D = 128
    ctx_pool = [1, 16, 17, 512, 511, 300, 1000, 33, 64, 129, 700, 2, 48, 250, 999, 15]
    ctx = ctx_pool[:B]
    rng = np.random.default_rng(300 + 7 * B + splits + NH + NKV)
    max_blocks = (max(ctx) + 15) // 16
    nb = B * max_blocks + 3
    tables = rng.permutation(nb)[:B * max_blocks].astype(np.int32).reshape(B, max_blocks)
    if B >= 4:
        b = 3                                           # the new token's block id is invalid
        tables[b, (ctx[b] - 1) // 16] = -1
    N = (NH + 2 * NKV) * D
    part = (rng.standard_normal((splits, B, N)) * 2).astype(np.float32)
    ck0, cv0 = rand_bf16(rng, (nb, NKV, 16, D)), rand_bf16(rng, (nb, NKV, D, 16))
    inv = torch.from_numpy(od.inv_freq(D, 500000.0, LLAMA3)).to(cuda)
    ctx_t = torch.tensor(ctx, dtype=torch.int32, device=cuda)
    tab = torch.from_numpy(tables).to(cuda)
    part_d = torch.from_numpy(part).to(cuda)
    scale = 1.0 / math.sqrt(D)
    print(f"fused rope+attention B={B} splits={splits} heads={NH}/{NKV} ctx={ctx}", flush=True)
    ck_a, cv_a = to_dev(ck0), to_dev(cv0)
    q = K.rope_cache_append_partials(part_d, inv, ctx_t, tab, ck_a, cv_a, NH)
    out_a = K.decode_attention(q, ck_a, cv_a, tab, ctx_t, max(ctx), scale=scale)
    ck_b, cv_b = to_dev(ck0), to_dev(cv0)
    out_b = K.decode_attention_rope(part_d, inv, ck_b, cv_b, tab, ctx_t, max(ctx), NH,
                                    scale=scale)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(to_host(out_b), to_host(out_a))
    np.testing.assert_array_equal(to_host(ck_b), to_host(ck_a))
    np.testing.assert_array_equal(to_host(cv_b), to_host(cv_a))


def test_fused_rope_attention_batch_invariant(cuda):
    """With plan_batch 16, the fused path at B=16 and at B=4 (the first four
    streams) runs the same context split but shares each unit differently (V
    halves only, or also 1 query head per workgroup): the four streams' outputs
    and cache contents are bit for bit the same, at contexts of one and of two
    context splits."""
    from rngd_pd_amd import kernels as K
    D, NH, NKV, splits = 128, 32, 8, 2
    for ctx in ([512, 300, 17, 511] * 4, [2048, 1500, 700, 1] * 4):
        rng = np.random.default_rng(77 + len(ctx) + ctx[0])
        max_blocks = (max(ctx) + 15) // 16
        nb = 16 * max_blocks + 3
        tables = rng.permutation(nb)[:16 * max_blocks].astype(np.int32).reshape(16, max_blocks)
        N = (NH + 2 * NKV) * D
        part = (rng.standard_normal((splits, 16, N)) * 2).astype(np.float32)
        ck0, cv0 = rand_bf16(rng, (nb, NKV, 16, D)), rand_bf16(rng, (nb, NKV, D, 16))
        inv = torch.from_numpy(od.inv_freq(D, 500000.0, LLAMA3)).to(cuda)
        outs, caches = [], []
        for B in (16, 4):
            print(f"fused rope batch invariance: B={B} max ctx {max(ctx)}", flush=True)
            ck, cv = to_dev(ck0), to_dev(cv0)
            out = K.decode_attention_rope(
                torch.from_numpy(np.ascontiguousarray(part[:, :B])).to(cuda), inv, ck, cv,
                torch.from_numpy(np.ascontiguousarray(tables[:B])).to(cuda),
                torch.tensor(ctx[:B], dtype=torch.int32, device=cuda), max(ctx), NH,
                scale=1.0 / math.sqrt(D), plan_batch=16)
            torch.cuda.synchronize()
            outs.append(to_host(out))
            caches.append((to_host(ck), to_host(cv)))
        np.testing.assert_array_equal(outs[1], outs[0][:4])
        # the cache blocks of streams 0-3 hold the same new tokens
        own = tables[:4].ravel()
        own = own[own >= 0]
        np.testing.assert_array_equal(caches[1][0][own], caches[0][0][own])
        np.testing.assert_array_equal(caches[1][1][own], caches[0][1][own])


def _rand_ssq(rng, n_tiles, B):
    """[B, n_tiles] per-tile sums of squares of plausible residual rows."""
    return (rng.chisquare(16, (B, n_tiles)) * rng.uniform(0.1, 3.0, (B, 1))).astype(np.float32)


def _host_rms(ssq, K, eps):
    """The row scale in fp64 (the kernels sum in fp32 in a fixed order)."""
    return 1.0 / np.sqrt(ssq.astype(np.float64).sum(1) / K + eps)


@pytest.mark.parametrize("splits", [1, 2, 4])
def test_rope_from_partials_with_row_scale(cuda, splits):
    """With the pre-attention norm folded, each row's summed partials are
    scaled by the row's r before the one rounding: q, the cache's new k and v
    equal rope_cache_append on bf16(r * sum) rows, within the fp32 rounding of
    r (compared exactly on the rows the kernel's r reproduces)."""
    from rngd_pd_amd import kernels as K
    NH, NKV, D, H = 8, 2, 128, 4096
    positions = [0, 17, 511, 4000]
    B = len(positions)
    rng = np.random.default_rng(700 + splits)
    max_blocks = max(positions) // 16 + 1
    nb = 2 * B + 1
    tables = np.zeros((B, max_blocks), np.int32)
    own = rng.permutation(np.arange(1, nb))[:B]
    for b, p in enumerate(positions):
        tables[b, p // 16] = own[b]
    N = (NH + 2 * NKV) * D
    part = (rng.standard_normal((splits, B, N)) * 3).astype(np.float32)
    ssq = _rand_ssq(rng, H // 16, B)
    eps = 1e-5
    total = part[0].copy()
    for s in range(1, splits):
        total = total + part[s]
    r = _host_rms(ssq, H, eps).astype(np.float32)
    ck0, cv0 = rand_bf16(rng, (nb, NKV, 16, D)), rand_bf16(rng, (nb, NKV, D, 16))
    inv = torch.from_numpy(od.inv_freq(D, 500000.0, LLAMA3)).to(cuda)
    ctx = torch.tensor([p + 1 for p in positions], dtype=torch.int32, device=cuda)
    tab = torch.from_numpy(tables).to(cuda)
    print(f"rope partials with row scale, splits={splits}", flush=True)
    ck_a, cv_a = to_dev(ck0), to_dev(cv0)
    K.rope_cache_append_partials(torch.from_numpy(part).to(cuda), inv, ctx, tab, ck_a, cv_a, NH,
                                 ssq=torch.from_numpy(ssq).to(cuda), eps=eps)
    torch.cuda.synchronize()
    got_v = _f32(to_host(cv_a))
    for b, p in enumerate(positions):
        want = (total[b, (NH + NKV) * D:] * r[b]).reshape(NKV, D)
        np.testing.assert_allclose(got_v[own[b], :, :, p % 16], want, rtol=2 * HALF_ULP, atol=0)


@pytest.mark.parametrize("B,splits,H", [(16, 2, 4096), (4, 2, 4096), (5, 4, 512), (1, 1, 8192)])
def test_fused_rope_attention_with_row_scale_equals_two_calls(cuda, B, splits, H):
    """pdk_decode_attn_rope_rms against pdk_rope_cache_append_partials_rms
    followed by pdk_decode_attn: bit-identical outputs and cache contents (the
    two compute each row's scale in the same fixed order)."""
    from rngd_pd_amd import kernels as K
    NH, NKV, D = 32, 8, 128
    ctx = [1, 16, 17, 512, 511, 300, 1000, 33, 64, 129, 700, 2, 48, 250, 999, 15][:B]
    rng = np.random.default_rng(900 + B + splits + H)
    max_blocks = (max(ctx) + 15) // 16
    nb = B * max_blocks + 3
    tables = rng.permutation(nb)[:B * max_blocks].astype(np.int32).reshape(B, max_blocks)
    N = (NH + 2 * NKV) * D
    part_d = torch.from_numpy((rng.standard_normal((splits, B, N)) * 2).astype(np.float32)).to(cuda)
    ssq = torch.from_numpy(_rand_ssq(rng, H // 16, B)).to(cuda)
    ck0, cv0 = rand_bf16(rng, (nb, NKV, 16, D)), rand_bf16(rng, (nb, NKV, D, 16))
    inv = torch.from_numpy(od.inv_freq(D, 500000.0, LLAMA3)).to(cuda)
    ctx_t = torch.tensor(ctx, dtype=torch.int32, device=cuda)
    tab = torch.from_numpy(tables).to(cuda)
    scale = 1.0 / math.sqrt(D)
    print(f"fused rope+attention with row scale B={B} splits={splits} H={H}", flush=True)
    ck_a, cv_a = to_dev(ck0), to_dev(cv0)
    q = K.rope_cache_append_partials(part_d, inv, ctx_t, tab, ck_a, cv_a, NH, ssq=ssq, eps=1e-5)
    out_a = K.decode_attention(q, ck_a, cv_a, tab, ctx_t, max(ctx), scale=scale)
    ck_b, cv_b = to_dev(ck0), to_dev(cv0)
    out_b = K.decode_attention_rope(part_d, inv, ck_b, cv_b, tab, ctx_t, max(ctx), NH,
                                    scale=scale, ssq=ssq, eps=1e-5)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(to_host(out_b), to_host(out_a))
    np.testing.assert_array_equal(to_host(ck_b), to_host(ck_a))
    np.testing.assert_array_equal(to_host(cv_b), to_host(cv_a))


@pytest.mark.parametrize("B,K,N,splits", [(16, 4096, 6144, 2), (4, 4096, 6144, 2),
                                          (3, 512, 1536, 1), (40, 1024, 512, 4)])
def test_linear_splitk_rms(cuda, B, K, N, splits):
    """The q|k|v projection after the folded pre-attention norm: each row's
    partials are the plain split-K partials times the row's r (the same fp32
    sums, one more product), tiled and untiled alike."""
    from rngd_pd_amd import kernels as K_
    rng = np.random.default_rng(B * 3 + K + N + splits)
    x, w = rand_bf16(rng, (B, K), 2.0), rand_bf16(rng, (N, K), 0.05)
    ssq = _rand_ssq(rng, K // 16, B)
    eps = 1e-5
    xd, wd, sd = to_dev(x), to_dev(w), torch.from_numpy(ssq).to(cuda)
    print(f"linear_splitk_rms B={B} K={K} N={N} splits={splits}", flush=True)
    plain = K_.linear_splitk(xd, wd, splits)
    got = K_.linear_splitk_rms(xd, wd, splits, sd, eps)
    got_t = K_.linear_splitk_rms(xd, K_.tile_weight(wd), splits, sd, eps)
    torch.cuda.synchronize()
    assert torch.equal(got, got_t)
    r = _host_rms(ssq, K, eps)
    np.testing.assert_allclose(got.cpu().numpy(), plain.cpu().numpy() * r[None, :, None],
                               rtol=2e-6, atol=1e-30)


@pytest.mark.parametrize("B,H", [(16, 4096), (3, 512), (64, 8192), (1, 16)])
def test_row_ssq(cuda, B, H):
    from rngd_pd_amd import kernels as K
    rng = np.random.default_rng(B + H)
    x = rand_bf16(rng, (B, H), 3.0)
    print(f"row_ssq B={B} H={H}", flush=True)
    got = K.row_ssq(to_dev(x)).cpu().numpy()
    want = (_f32(x).astype(np.float64).reshape(B, H // 16, 16) ** 2).sum(-1)
    np.testing.assert_allclose(got, want, rtol=1e-6)


@pytest.mark.parametrize("tok_dtype", [torch.int32, torch.int64])
def test_embed_ssq(cuda, tok_dtype):
    """The fused lookup: x equal to the table's rows bit for bit (a zero row for
    ids outside [0, vocab)), ssq bit-identical to row_ssq of that x."""
    from rngd_pd_amd import kernels as K
    rng = np.random.default_rng(5)
    V, H, B = 1000, 4096, 16
    table = to_dev(rand_bf16(rng, (V, H), 2.0))
    ids = rng.integers(0, V, B)
    ids[3], ids[7], ids[11] = -1, V, 0          # out of range both ways, and the first row
    tok = torch.from_numpy(ids).to(cuda).to(tok_dtype)
    print(f"embed_ssq tokens {tok_dtype}", flush=True)
    x, ssq = K.embed_ssq(table, tok)
    torch.cuda.synchronize()
    want = to_host(table)[np.clip(ids, 0, V - 1)].copy()
    want[(ids < 0) | (ids >= V)] = 0
    np.testing.assert_array_equal(to_host(x), want)
    ref = K.row_ssq(to_dev(want))
    assert torch.equal(ssq, ref)


@pytest.mark.parametrize("B,K,N,splits", [(16, 14336, 4096, 4), (4, 14336, 4096, 4),
                                          (3, 1024, 512, 8), (33, 512, 2048, 2), (1, 128, 16, 1)])
def test_linear_splitk_final(cuda, B, K, N, splits):
    """The down projection with the residual add of the next norm: residual
    bit-identical to linear_splitk + rmsnorm_partials' update, ssq the sums
    of squares of the result, the counters back at zero, and the same on a
    second call and on tiled weights."""
    from rngd_pd_amd import kernels as K_
    rng = np.random.default_rng(B * 5 + K + N + splits)
    w = rand_bf16(rng, (N, K), 0.05)
    wd = to_dev(w)
    counters = torch.zeros(N // 16, dtype=torch.int32, device=cuda)
    ones = torch.ones(N, dtype=BF16, device=cuda)
    print(f"linear_splitk_final B={B} K={K} N={N} splits={splits}", flush=True)
    for call, wgt in enumerate((wd, K_.tile_weight(wd), wd)):
        x, r = rand_bf16(rng, (B, K)), rand_bf16(rng, (B, N), 4.0)
        xd = to_dev(x)
        want = to_dev(r)
        parts = K_.linear_splitk(xd, wd, splits)
        K_.rmsnorm_partials(want, parts, splits, ones, 1e-5)
        got = to_dev(r)
        ssq = torch.full((B, N // 16), float("nan"), dtype=torch.float32, device=cuda)
        K_.linear_splitk_final(xd, wgt, splits, got, ssq, counters)
        torch.cuda.synchronize()
        assert torch.equal(got.view(torch.int16), want.view(torch.int16)), call
        gf = _f32(to_host(got)).astype(np.float64)
        np.testing.assert_allclose(ssq.cpu().numpy(), (gf.reshape(B, N // 16, 16) ** 2).sum(-1),
                                   rtol=1e-6, atol=1e-30)
        assert int(counters.abs().sum()) == 0, call


@pytest.mark.parametrize("B,K,N", [(16, 4096, 128256), (4, 4096, 128256), (3, 256, 1000)])
def test_linear_argmax_rms(cuda, B, K, N):
    """The lm_head on weights folded with the final norm's gain: logits within
    half an ulp of r * (x . w'^T) in fp64, tokens the first maximum of those
    bf16 logits (pdk_greedy_argmax on the same logits)."""
    from rngd_pd_amd import kernels as K_
    rng = np.random.default_rng(B + K + N + 1)
    x, w = rand_bf16(rng, (B, K), 2.0), rand_bf16(rng, (N, K), 0.05)
    ssq = _rand_ssq(rng, K // 16, B)
    eps = 1e-5
    wd = to_dev(w)
    keys = torch.zeros(B, dtype=torch.int64, device=cuda)
    logits = torch.empty((B, N), dtype=BF16, device=cuda)
    print(f"linear_argmax_rms B={B} K={K} N={N}", flush=True)
    wt = K_.tile_weight(wd)
    tok = K_.linear_argmax_rms(to_dev(x), wt, torch.from_numpy(ssq).to(cuda), eps,
                               keys, logits=logits)
    want_tok = K_.greedy_argmax(logits)
    torch.cuda.synchronize()
    assert torch.equal(tok.cpu(), want_tok.cpu().to(torch.int32))
    assert int(keys.abs().sum()) == 0
    r = _host_rms(ssq, K, eps)
    ref = (_f32(x).astype(np.float64) @ _f32(w).astype(np.float64).T) * r[:, None]
    np.testing.assert_allclose(_f32(to_host(logits)), ref, rtol=HALF_ULP, atol=1e-3 * np.abs(ref).max())


@pytest.mark.parametrize("B,M", [(3, 14336), (1, 8), (16, 1024)])
def test_swiglu(cuda, B, M):
    from rngd_pd_amd import kernels as K
    rng = np.random.default_rng(M + B)
    gu = rand_bf16(rng, (B, 2 * M), 4.0)
    gu[0, :4] = _bf16_bits_rne(np.array([100.0, -100.0, 0.0, -0.0], np.float32))
    print(f"swiglu B={B} M={M}", flush=True)
    out = K.swiglu(to_dev(gu))
    torch.cuda.synchronize()
    got = _f32(to_host(out))
    assert np.isfinite(got).all()
    np.testing.assert_allclose(got, od.swiglu(_f32(gu)), rtol=HALF_ULP, atol=1e-6)


@pytest.mark.parametrize("B,K,N", [(1, 128, 16), (4, 4096, 6144), (16, 14336, 4096),
                                   (17, 512, 48), (33, 1024, 256), (64, 256, 32),
                                   (5, 256, 1000), (2, 128, 7)])
def test_linear(cuda, B, K, N):
    """y = x . w^T, then y = r + x . w^T in place: fp32 sums, one bf16 rounding."""
    from rngd_pd_amd import kernels as K_
    rng = np.random.default_rng(B * 1000 + N)
    x, w, r = rand_bf16(rng, (B, K)), rand_bf16(rng, (N, K), 0.05), rand_bf16(rng, (B, N), 4.0)
    xd, wd, rd = to_dev(x), to_dev(w), to_dev(r)
    print(f"linear B={B} K={K} N={N}", flush=True)
    y = K_.linear(xd, wd)
    K_.linear(xd, wd, residual=rd, out=rd)
    torch.cuda.synchronize()
    want = _f32(x).astype(np.float64) @ _f32(w).astype(np.float64).T
    tol = 1e-5 * np.abs(want).max()                 # fp32 summation order
    np.testing.assert_allclose(_f32(to_host(y)), want, rtol=HALF_ULP, atol=tol)
    np.testing.assert_allclose(_f32(to_host(rd)), want + _f32(r), rtol=HALF_ULP, atol=tol)


@pytest.mark.parametrize("B,K,N,splits", [(16, 14336, 4096, 4), (4, 14336, 4096, 4),
                                          (3, 1024, 512, 8), (33, 384, 48, 3), (1, 128, 16, 1)])
def test_linear_splitk_and_rmsnorm_partials(cuda, B, K, N, splits):
    """Partial sums over the K split add up to x . w^T (fp32); the norm adds
    them to the residual in order, rounds once, and normalises."""
    from rngd_pd_amd import kernels as K_
    rng = np.random.default_rng(B * 7 + K + splits)
    x, w = rand_bf16(rng, (B, K)), rand_bf16(rng, (N, K), 0.05)
    r, g = rand_bf16(rng, (B, N), 4.0), rand_bf16(rng, (N,))
    print(f"linear_splitk B={B} K={K} N={N} splits={splits}", flush=True)
    part = K_.linear_splitk(to_dev(x), to_dev(w), splits)
    torch.cuda.synchronize()
    want = _f32(x).astype(np.float64) @ _f32(w).astype(np.float64).T
    got = part.cpu().numpy().astype(np.float64)
    np.testing.assert_allclose(got.sum(0), want, rtol=1e-5, atol=1e-5 * np.abs(want).max())
    steps = K // 128
    for s in range(splits):                                   # each split holds its own K range
        lo, hi = s * steps // splits * 128, (s + 1) * steps // splits * 128
        ws = _f32(x)[:, lo:hi].astype(np.float64) @ _f32(w)[:, lo:hi].astype(np.float64).T
        np.testing.assert_allclose(got[s], ws, rtol=1e-5, atol=1e-5 * np.abs(want).max() + 1e-6)
    if N % 8 == 0 and N >= 8:
        xd = to_dev(r)
        out = K_.rmsnorm_partials(xd, part, splits, to_dev(g), 1e-5)
        torch.cuda.synchronize()
        acc = np.zeros((B, N), np.float32)
        for s in range(splits):
            acc = acc + part[s].cpu().numpy()
        summed = _bf16_bits_rne(_f32(r) + acc)
        np.testing.assert_array_equal(to_host(xd), summed)
        np.testing.assert_allclose(_f32(to_host(out)), od.rmsnorm(_f32(summed), _f32(g), 1e-5),
                                   rtol=HALF_ULP, atol=1e-6)


@pytest.mark.parametrize("B,K,M", [(4, 4096, 14336), (16, 128, 16), (40, 512, 64), (3, 256, 24),
                                   (40, 256, 12288), (24, 256, 12288)])
def test_linear_swiglu(cuda, B, K, M):
    from rngd_pd_amd import kernels as K_
    rng = np.random.default_rng(B + K + M)
    x, w = rand_bf16(rng, (B, K)), rand_bf16(rng, (2 * M, K), 0.05)
    print(f"linear_swiglu B={B} K={K} M={M}", flush=True)
    y = K_.linear_swiglu(to_dev(x), to_dev(w))
    torch.cuda.synchronize()
    gu = _f32(x).astype(np.float64) @ _f32(w).astype(np.float64).T
    want = od.swiglu(gu)
    tol = 1e-5 * np.abs(gu).max() ** 2
    np.testing.assert_allclose(_f32(to_host(y)), want, rtol=HALF_ULP, atol=tol)


@pytest.mark.parametrize("B,K,N", [(16, 4096, 4096), (4, 4096, 4096), (16, 14336, 4096),
                                   (3, 256, 1024), (64, 128, 256), (1, 128, 16), (33, 512, 2048)])
def test_linear_ssq(cuda, B, K, N):
    """The O and down projections with the norm's raw material: y bit-identical to
    pdk_linear with the residual, ssq[t][b] the sum of y[b, 16t:16t+16]^2
    (as bf16 values), tiled and untiled weights alike."""
    from rngd_pd_amd import kernels as K_
    rng = np.random.default_rng(B * 7 + K + N)
    x, w, r = rand_bf16(rng, (B, K)), rand_bf16(rng, (N, K), 0.05), rand_bf16(rng, (B, N), 4.0)
    xd, wd = to_dev(x), to_dev(w)
    print(f"linear_ssq B={B} K={K} N={N}", flush=True)
    want_y = K_.linear(xd, wd, residual=to_dev(r))
    outs = []
    for wgt in (wd, K_.tile_weight(wd)):
        rd = to_dev(r)
        ssq = torch.full((B, N // 16), float("nan"), dtype=torch.float32, device=cuda)
        y = K_.linear_ssq(xd, wgt, rd, ssq, out=rd)            # in place, as the decoder runs it
        outs.append((y, ssq))
    torch.cuda.synchronize()
    for y, ssq in outs:
        assert torch.equal(y.view(torch.int16), want_y.view(torch.int16))
        yf = _f32(to_host(y)).astype(np.float64)
        want = (yf.reshape(B, N // 16, 16) ** 2).sum(-1)
        np.testing.assert_allclose(ssq.cpu().numpy(), want, rtol=1e-6, atol=1e-30)
    assert torch.equal(outs[0][1], outs[1][1])


@pytest.mark.parametrize("B,K,M", [(16, 4096, 14336), (4, 4096, 14336), (3, 256, 64),
                                   (40, 512, 64), (1, 128, 16)])
def test_linear_swiglu_rms(cuda, B, K, M):
    """gate|up of rmsnorm(x) * g from the un-normalised x, the gain folded into
    the weights and the row scale taken from per-tile sums of squares: within
    half an ulp of the same products in fp64 (the folded bf16 weights, the
    exact row scale), within 1 % of the unfused norm -> gate|up, and the
    same bits on tiled weights."""
    from rngd_pd_amd import kernels as K_
    rng = np.random.default_rng(B * 13 + K + M)
    x = rand_bf16(rng, (B, K), 2.0)
    w = rand_bf16(rng, (2 * M, K), 0.05)
    g = _bf16_bits_rne(1.0 + 0.1 * rng.standard_normal(K).astype(np.float32))
    eps = 1e-5
    xd, wd, gd = to_dev(x), to_dev(w), to_dev(g)
    xf = _f32(x).astype(np.float64)
    ssq = torch.from_numpy((xf.reshape(B, K // 16, 16) ** 2).sum(-1).astype(np.float32))
    ssq = ssq.contiguous().to(cuda)
    print(f"linear_swiglu_rms B={B} K={K} M={M}", flush=True)
    wf = K_.fold_norm(wd, gd)
    y = K_.linear_swiglu_rms(xd, wf, ssq, eps)
    y_t = K_.linear_swiglu_rms(xd, K_.tile_weight(wf), ssq, eps)
    # the unfused path: pdk_rmsnorm then pdk_linear_swiglu on the raw weights
    h = K_.rmsnorm(xd, gd, eps)
    y_ref = K_.linear_swiglu(h, wd)
    torch.cuda.synchronize()
    assert torch.equal(y.view(torch.int16), y_t.view(torch.int16))
    r = 1.0 / np.sqrt(ssq.cpu().numpy().astype(np.float64).sum(1) / K + eps)     # [B]
    gu = (xf @ _f32(to_host(wf)).astype(np.float64).T) * r[:, None]
    want = od.swiglu(gu)
    tol = 1e-5 * np.abs(gu).max() ** 2
    np.testing.assert_allclose(_f32(to_host(y)), want, rtol=HALF_ULP, atol=tol)
    a, b = _f32(to_host(y)).astype(np.float64), _f32(to_host(y_ref)).astype(np.float64)
    assert np.linalg.norm(a - b) <= 0.01 * np.linalg.norm(b)


@pytest.mark.parametrize("B,K,N", [(16, 4096, 128256), (4, 4096, 128256), (3, 256, 1000),
                                   (1, 128, 7)])
def test_linear_argmax(cuda, B, K, N):
    """The fused lm_head argmax equals pdk_greedy_argmax over the same bf16
    logits: duplicated weight rows make exact ties (the first column wins), a
    NaN row wins outright, and a second call sees the scratch left at zero."""
    from rngd_pd_amd import kernels as K_
    rng = np.random.default_rng(B + N)
    x, w = rand_bf16(rng, (B, K)), rand_bf16(rng, (N, K), 0.05)
    wd = to_dev(w)
    if N > 500:
        logits = K_.linear(to_dev(x), wd).float().cpu().numpy()
        top = int(np.argmax(logits[0]))
        wd[top - 3 if top >= 3 else top + 1].copy_(wd[top])          # a tie with row 0's best
        wd[N - 1].fill_(float("nan"))                               # NaN in every row
    keys = torch.zeros(B, dtype=torch.int64, device=cuda)
    xd = to_dev(x)
    print(f"linear_argmax B={B} K={K} N={N}", flush=True)
    for call in range(2):
        lg = torch.empty((B, N), dtype=torch.bfloat16, device=cuda)
        tok = K_.linear_argmax(xd, wd, keys, logits=lg)
        ref = K_.greedy_argmax(lg)
        torch.cuda.synchronize()
        assert torch.equal(keys, torch.zeros_like(keys))
        np.testing.assert_array_equal(tok.cpu().numpy(), ref.cpu().numpy())
        np.testing.assert_array_equal(to_host(lg), to_host(K_.linear(xd, wd)))
        if N > 500 and call == 0:
            assert (tok.cpu().numpy() == N - 1).all()
            wd[N - 1].zero_()                                      # second call: the tie decides
            torch.cuda.synchronize()
        elif N > 500:
            assert tok[0].item() == min(top - 3 if top >= 3 else top, top)
        else:
            xd = xd.flip(0).contiguous()


def _tiled_layout(w):
    """The documented tiled layout of a [N, K] weight, by reshapes: block (t, s)
    starts at (s * ceil(N/16) + t) * 2048 (step-major), and its element
    ((c*4 + kg)*16 + col)*8 + e = w[16t + col][128s + 32c + 8kg + e]."""
    N, K = w.shape
    nt = (N + 15) // 16
    pad = np.zeros((nt * 16, K), w.dtype)
    pad[:N] = w
    v = pad.reshape(nt, 16, K // 128, 4, 4, 8)            # t, col, s, c, kg, e
    return np.ascontiguousarray(v.transpose(2, 0, 3, 4, 1, 5)).reshape(-1)


@pytest.mark.parametrize("N,K", [(16, 128), (1000, 256), (7, 128), (6144, 4096), (128256, 128)])
def test_weight_tile_layout(cuda, N, K):
    from rngd_pd_amd import kernels as K_
    rng = np.random.default_rng(N + K)
    w = rand_bf16(rng, (N, K))
    print(f"weight_tile N={N} K={K}", flush=True)
    t = K_.tile_weight(to_dev(w))
    torch.cuda.synchronize()
    assert t.shape == (N, K)
    np.testing.assert_array_equal(to_host(t.data), _tiled_layout(w))


@pytest.mark.parametrize("B,K,N", [(1, 128, 16), (4, 4096, 6144), (16, 14336, 4096),
                                   (16, 4096, 4096), (33, 1024, 2048), (5, 256, 1000),
                                   (64, 256, 32), (2, 128, 7), (4, 128, 70000),
                                   (16, 256, 28672), (24, 256, 24576), (40, 128, 131072)])
def test_tiled_gemms_equal_untiled(cuda, B, K, N):
    """Every GEMM entry point gives bit-identical results on the tiled copy of
    its weight: the same products, summed in the same order."""
    from rngd_pd_amd import kernels as K_
    rng = np.random.default_rng(B * 31 + K + N)
    x, w, r = rand_bf16(rng, (B, K)), rand_bf16(rng, (N, K), 0.05), rand_bf16(rng, (B, N), 4.0)
    xd, wd, rd = to_dev(x), to_dev(w), to_dev(r)
    wt = K_.tile_weight(wd)
    print(f"tiled gemms B={B} K={K} N={N}", flush=True)
    pairs = [(K_.linear(xd, wd), K_.linear(xd, wt)),
             (K_.linear(xd, wd, residual=rd), K_.linear(xd, wt, residual=rd))]
    for splits in sorted({1, min(4, K // 128)}):
        pairs.append((K_.linear_splitk(xd, wd, splits), K_.linear_splitk(xd, wt, splits)))
    keys = torch.zeros(B, dtype=torch.int64, device=cuda)
    pairs.append((K_.linear_argmax(xd, wd, keys), K_.linear_argmax(xd, wt, keys)))
    if N % 32 == 0:                                   # gate|up: 2M rows with M % 16 == 0
        pairs.append((K_.linear_swiglu(xd, wd), K_.linear_swiglu(xd, wt)))
    torch.cuda.synchronize()
    for i, (a, b) in enumerate(pairs):
        assert torch.equal(a.view(torch.int16) if a.dtype == torch.bfloat16 else a,
                           b.view(torch.int16) if b.dtype == torch.bfloat16 else b), i


def test_tiled_swiglu_needs_m_multiple_of_16(cuda):
    from rngd_pd_amd import kernels as K_
    from rngd_pd_amd._lib import PdkError
    rng = np.random.default_rng(5)
    x, w = rand_bf16(rng, (2, 128)), rand_bf16(rng, (2 * 24, 128))
    wt = K_.tile_weight(to_dev(w))
    with pytest.raises(PdkError, match="M % 16"):
        K_.linear_swiglu(to_dev(x), wt)


# ---- whole steps -------------------------------------------------------------

class _OCfg:
    def __init__(self, cfg):
        self.n_heads, self.n_kv_heads, self.eps = cfg.n_heads, cfg.n_kv_heads, cfg.eps
        self.inv = cfg.inv_freq().numpy()


def _oracle_weights(w):
    """The engine's [out, in] bf16 weights as the oracle's [in, out] float32."""
    f = lambda t: t.float().cpu().numpy()   # noqa: E731
    T = lambda t: np.ascontiguousarray(f(t).T)   # noqa: E731
    return {"embed": f(w.embed), "norm_f": f(w.norm_f), "lm_head": T(w.lm_head),
            "layers": [(f(w.norm1[i]), T(w.wqkv[i]), T(w.wo[i]), f(w.norm2[i]), T(w.wgu[i]),
                        T(w.wd[i])) for i in range(w.cfg.n_layers)]}


def _prefilled(cuda, cfg, ctx, steps, rng):
    """A paged cache whose streams hold random KV at positions 0..ctx[b]-2 (the
    step writes ctx[b]-1), with the same values in dense oracle caches."""
    from rngd_pd_amd.engines.paged_cache import PagedKVCache
    B, L, NKV, HD = len(ctx), cfg.n_layers, cfg.n_kv_heads, cfg.head_dim
    S = max(ctx) + steps
    per = (S + 15) // 16
    nb = B * per + 3
    tables = rng.permutation(nb)[:B * per].astype(np.int32).reshape(B, per)
    cache = PagedKVCache(L, nb, NKV, HD, device=cuda)
    Ks, Vs = [], []
    have = [c - 1 for c in ctx]
    for li in range(L):
        k = rand_bf16(rng, (B, NKV, S, HD))
        v = rand_bf16(rng, (B, NKV, S, HD))
        for b, h in enumerate(have):
            k[b, :, h:] = 0
            v[b, :, h:] = 0
        ck, cv = oatt.paged_from_dense(np.transpose(k, (0, 1, 3, 2)), v, have, tables, nb)
        cache.k[li].copy_(to_dev(ck))
        cache.v[li].copy_(to_dev(cv))
        Ks.append(_f32(k))
        Vs.append(_f32(v))
    return cache, torch.from_numpy(tables).to(cuda), Ks, Vs


def _check_step(dec, B, want_tok, want_x, want_logits, label):
    got_x = dec.x[:B].float().cpu().numpy()
    got_logits = dec.logits[:B].float().cpu().numpy()
    got_tok = dec.tokens[:B].cpu().numpy()
    rel = od.rel_l2(got_x, want_x)
    rel_logits = od.rel_l2(got_logits, want_logits)
    print(f"{label}: hidden rel {rel:.5f} logits rel {rel_logits:.5f}", flush=True)
    assert rel < REL_REFERENCE_BAR, f"{label}: hidden rel {rel}"
    assert rel < REL_TIGHT, f"{label}: hidden rel {rel}"
    assert rel_logits < REL_TIGHT, f"{label}: logits rel {rel_logits}"
    np.testing.assert_array_equal(got_tok, np.argmax(got_logits, -1))   # first maximum
    checked = 0
    for b in range(B):
        top2 = np.sort(want_logits[b])[-2:]
        err = np.abs(got_logits[b] - want_logits[b]).max()
        if top2[1] - top2[0] > 2 * err:
            assert got_tok[b] == want_tok[b], f"{label}: stream {b} token"
            checked += 1
    return got_tok, checked


def _run_steps(cuda, cfg, ctx, steps, seed):
    from rngd_pd_amd.engines.llama_decode import LlamaDecoder, LlamaWeights
    rng = np.random.default_rng(seed)
    B = len(ctx)
    w = LlamaWeights.random(cfg, seed=seed, device=cuda)
    ow, ocfg = _oracle_weights(w), _OCfg(cfg)
    cache, tables, Ks, Vs = _prefilled(cuda, cfg, ctx, steps, rng)
    dec = LlamaDecoder(w, cache, max_batch=B)
    tok = rng.integers(0, cfg.vocab, B)
    checked = 0
    for s in range(steps):
        pos = [c - 1 + s for c in ctx]
        ctx_d = torch.tensor([p + 1 for p in pos], dtype=torch.int32, device=cuda)
        dec.step(torch.from_numpy(tok).to(cuda), ctx_d, tables, max(pos) + 1)
        torch.cuda.synchronize()
        want_tok, want_x, want_logits = od.decode_step(tok, ow, Ks, Vs, pos, ocfg)
        got_tok, n = _check_step(dec, B, want_tok, want_x, want_logits, f"step {s}")
        checked += n
        tok = got_tok.astype(np.int64)                # both sides continue from the same tokens
    assert checked >= steps * B // 2, f"only {checked} tokens had a clear margin"
    return dec


def test_small_model_steps(cuda):
    from rngd_pd_amd.engines.llama_decode import LlamaConfig
    cfg = LlamaConfig(hidden=512, n_heads=8, n_kv_heads=2, head_dim=128, inter=1024,
                      vocab=1000, n_layers=3)
    print("small model: 3 layers, ctx [1, 16, 17, 200, 513]", flush=True)
    _run_steps(cuda, cfg, [1, 16, 17, 200, 513], steps=3, seed=11)


def test_small_model_steps_two_row_tiles(cuda):
    """B = 20: every GEMM runs two 16-row tiles (the residual loaded early for
    both, the prefetch depth of the two-tile shapes)."""
    from rngd_pd_amd.engines.llama_decode import LlamaConfig
    cfg = LlamaConfig(hidden=512, n_heads=8, n_kv_heads=2, head_dim=128, inter=1024,
                      vocab=1000, n_layers=2)
    ctx = [1, 16, 17, 200, 513, 64, 5, 300, 129, 2, 40, 77, 256, 511, 100, 33, 18, 250, 3, 90]
    print("small model: 2 layers, B=20", flush=True)
    _run_steps(cuda, cfg, ctx, steps=2, seed=13)


def test_llama8b_shape_two_layers(cuda):
    """Llama-3.1-8B dimensions (hidden 4096, 32/8 heads, MLP 14336, vocab
    128256) with 2 of the 32 layers, B=16 at mixed context lengths."""
    from rngd_pd_amd.engines.llama_decode import LlamaConfig
    cfg = LlamaConfig(n_layers=2)
    ctx = [512, 1, 511, 300, 17, 16, 64, 129, 512, 2, 480, 33, 256, 99, 400, 512]
    print("llama-8b shape: 2 layers, B=16", flush=True)
    _run_steps(cuda, cfg, ctx, steps=2, seed=5)


def test_graph_replays_match_eager(cuda):
    """The step captured as a HIP graph replays the eager result, with eager
    work and synchronisation between replays."""
    from rngd_pd_amd.engines.llama_decode import LlamaConfig, LlamaDecoder, LlamaWeights
    cfg = LlamaConfig(hidden=512, n_heads=8, n_kv_heads=2, head_dim=128, inter=1024,
                      vocab=1000, n_layers=2)
    rng = np.random.default_rng(3)
    ctx = [40, 300, 7, 129]
    B = len(ctx)
    w = LlamaWeights.random(cfg, seed=3, device=cuda)
    cache, tables, _, _ = _prefilled(cuda, cfg, ctx, 1, rng)
    dec = LlamaDecoder(w, cache, max_batch=B)
    tok = torch.from_numpy(rng.integers(0, cfg.vocab, B)).to(cuda)
    ctx_d = torch.tensor(ctx, dtype=torch.int32, device=cuda)
    cap = tables.shape[1] * 16
    print("graph capture: 2 layers, B=4", flush=True)
    dec.step(tok, ctx_d, tables, cap)
    torch.cuda.synchronize()
    want_x, want_tok = dec.x[:B].clone(), dec.tokens[:B].clone()
    graph = dec.capture(tok, ctx_d, tables, cap)
    for r in range(3):
        dec.x_buf.zero_()
        dec.tokens.fill_(-1)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        rel = od.rel_l2(dec.x[:B].float().cpu().numpy(), want_x.float().cpu().numpy())
        print(f"replay {r}: rel {rel:.2e}", flush=True)
        assert rel < 1e-3
        assert torch.equal(dec.tokens[:B], want_tok)
        _ = torch.randn(1000, device=cuda).sum().item()           # eager work between replays


def _small_decoder(cuda, n_layers=2, max_batch=8, plan_batch=None, width_blocks=128, seed=21):
    from rngd_pd_amd.engines.llama_decode import LlamaConfig, LlamaDecoder, LlamaWeights
    from rngd_pd_amd.engines.paged_cache import PagedKVCache
    cfg = LlamaConfig(hidden=512, n_heads=8, n_kv_heads=2, head_dim=128, inter=1024,
                      vocab=1000, n_layers=n_layers)
    w = LlamaWeights.random(cfg, seed=seed, device=cuda)
    nb = max_batch * width_blocks + 3
    cache = PagedKVCache(n_layers, nb, cfg.n_kv_heads, cfg.head_dim, device=cuda)
    gen = torch.Generator(device=cuda).manual_seed(seed)
    for li in range(n_layers):
        cache.k[li].copy_(torch.randn(cache.k[li].shape, generator=gen, device=cuda))
        cache.v[li].copy_(torch.randn(cache.v[li].shape, generator=gen, device=cuda))
    perm = np.random.default_rng(seed).permutation(nb)[:max_batch * width_blocks]
    tables = torch.from_numpy(perm.astype(np.int32).reshape(max_batch, width_blocks)).to(cuda)
    dec = LlamaDecoder(w, cache, max_batch=max_batch, plan_batch=plan_batch)
    return cfg, dec, tables


def test_batch_invariant_step(cuda):
    """With a fixed plan batch a stream's step is bit for bit the same alone
    (B = 1) as in row 3 of a batch of 8, at contexts the attention splits."""
    cfg, dec, tables = _small_decoder(cuda, max_batch=8)
    rng = np.random.default_rng(4)
    ctx = torch.tensor([600, 31, 1200, 777, 5, 2047, 64, 900], dtype=torch.int32, device=cuda)
    tok = torch.from_numpy(rng.integers(0, cfg.vocab, 8)).to(cuda)
    max_ctx = tables.shape[1] * 16
    print("batch invariance: B=8 then row 3 alone", flush=True)
    dec.step(tok, ctx, tables, max_ctx)
    torch.cuda.synchronize()
    want_x, want_tok = dec.x[3].clone(), int(dec.tokens[3])
    dec.step(tok[3:4], ctx[3:4], tables[3:4].contiguous(), max_ctx)
    torch.cuda.synchronize()
    assert torch.equal(dec.x[0].view(torch.int16), want_x.view(torch.int16))
    assert int(dec.tokens[0]) == want_tok


def test_workspace_never_grows_under_a_graph(cuda):
    """A graph captured where attention needs no workspace keeps no address for
    one: a later step that would allocate it raises instead of leaving the
    graph pointing at freed memory; reserve() first makes both work."""
    cfg, dec, tables = _small_decoder(cuda, max_batch=4)
    tables = tables[:4].contiguous()
    B = 4
    tok = torch.zeros(B, dtype=torch.int64, device=cuda)
    short = torch.full((B,), 60, dtype=torch.int32, device=cuda)
    long = torch.full((B,), 2000, dtype=torch.int32, device=cuda)
    print("workspace under a graph", flush=True)
    graph = dec.capture(tok, short, tables, 64)
    graph.replay()
    torch.cuda.synchronize()
    with pytest.raises(RuntimeError, match="reserve"):
        dec.step(tok, long, tables, 2048)
    cfg, dec2, tables2 = _small_decoder(cuda, max_batch=4)
    tables2 = tables2[:4].contiguous()
    dec2.reserve(2048)
    graph2 = dec2.capture(tok, short, tables2, 64)
    dec2.step(tok, long, tables2, 2048)
    graph2.replay()
    torch.cuda.synchronize()
