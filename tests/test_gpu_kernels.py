"""Parity of the HIP kernels (through the C ABI) against the CPU oracle.

Handoff kernels are permutations of bf16 bits: bit-exact. Decode attention is
floating point: bf16 outputs within 2e-2 abs / 1e-2 rel of the fp32 check
(the tolerance the decode path is specified to).
"""
import math

import numpy as np
import pytest
import torch

from oracle import native as orc
from tests._util import rand_bf16, to_dev, to_host

pytestmark = pytest.mark.gpu

ATOL, RTOL = 2e-2, 1e-2


def _prefill(rng, L, T, H, D):
    return rand_bf16(rng, (L, T, H, D)), rand_bf16(rng, (L, T, H, D))


@pytest.mark.parametrize("L,T,S,P,H,D", [
    (2, 16, 16, 16, 8, 128),
    (2, 64, 64, 37, 8, 128),
    (3, 100, 128, 100, 8, 128),
    (1, 512, 512, 512, 8, 128),
    (2, 512, 512, 0, 8, 128),
    (4, 300, 512, 300, 8, 128),
    (2, 80, 80, 65, 2, 64),
    (32, 512, 512, 257, 8, 128),
])
def test_pack_bit_exact(cuda, L, T, S, P, H, D):
    from rngd_pd_amd.kernels import pack_kv
    rng = np.random.default_rng(L * 1000 + P)
    k, v = _prefill(rng, L, T, H, D)
    want = orc.pack_kv(k, v, P, S)
    frame = pack_kv(to_dev(k), to_dev(v), P, S)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(to_host(frame), want)


def test_pack_strided_stack(cuda):
    """A stacked [L, 2, T, Hkv, D] prefill tensor packs through kv[:, 0] / kv[:, 1]."""
    from rngd_pd_amd.kernels import pack_kv
    rng = np.random.default_rng(7)
    L, T, H, D, S, P = 4, 96, 8, 128, 128, 90
    kv = rand_bf16(rng, (L, 2, T, H, D))
    want = orc.pack_kv(kv[:, 0], kv[:, 1], P, S)
    d = to_dev(kv)
    frame = pack_kv(d[:, 0], d[:, 1], P, S)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(to_host(frame), want)


def test_pack_batch(cuda):
    from rngd_pd_amd.kernels import pack_kv_batch, frame_shape
    rng = np.random.default_rng(11)
    L, H, D, S = 3, 8, 128, 512
    Ps = [64, 511, 1, 512, 200]
    reqs, wants = [], []
    for P in Ps:
        k, v = _prefill(rng, L, S, H, D)
        wants.append(orc.pack_kv(k, v, P, S))
        frame = torch.full(frame_shape(L, H, D, S), 7.0, dtype=torch.bfloat16, device=cuda)
        reqs.append((to_dev(k), to_dev(v), P, frame))
    pack_kv_batch(reqs, S)
    torch.cuda.synchronize()
    for (_, _, _, frame), want in zip(reqs, wants):
        np.testing.assert_array_equal(to_host(frame), want)


def _cache(L, nb, H, D, fill=0x3F80):
    ck = np.full((L, nb, H, 16, D), fill, np.uint16)
    cv = np.full((L, nb, H, D, 16), fill, np.uint16)
    return ck, cv


@pytest.mark.parametrize("L,S,P,H,D", [
    (2, 16, 16, 8, 128),
    (2, 64, 37, 8, 128),
    (3, 512, 512, 8, 128),
    (2, 512, 1, 8, 128),
    (2, 512, 0, 8, 128),
    (32, 512, 333, 8, 128),
    (2, 96, 81, 2, 64),
])
def test_scatter_bit_exact(cuda, L, S, P, H, D):
    from rngd_pd_amd.kernels import scatter_paged
    rng = np.random.default_rng(P + 5)
    k, v = _prefill(rng, L, S, H, D)
    frame = orc.pack_kv(k, v, P, S)
    nb = max(1, (S // 16) * 2)
    table = rng.permutation(nb)[: max(1, (P + 15) // 16)].astype(np.int32)
    ck, cv = _cache(L, nb, H, D)
    want_k, want_v = ck.copy(), cv.copy()
    orc.scatter_paged(frame, table, P, S, H, D, want_k, want_v)
    dk, dv = to_dev(ck), to_dev(cv)
    scatter_paged(to_dev(frame), table, P, S, dk, dv)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(to_host(dk), want_k)
    np.testing.assert_array_equal(to_host(dv), want_v)


def test_scatter_batch_and_gather_round_trip(cuda):
    from rngd_pd_amd.kernels import scatter_paged_batch, gather_paged
    rng = np.random.default_rng(3)
    L, S, H, D = 4, 512, 8, 128
    Ps = [int(p) for p in rng.integers(64, 513, 8)]
    need = [(p + 15) // 16 for p in Ps]
    nb = sum(need) + 5
    perm = rng.permutation(nb).astype(np.int32)
    tables, off = [], 0
    for n in need:
        tables.append(perm[off:off + n])
        off += n
    ck, cv = _cache(L, nb, H, D, fill=0)
    want_k, want_v = ck.copy(), cv.copy()
    frames = []
    for P, t in zip(Ps, tables):
        k, v = _prefill(rng, L, S, H, D)
        f = orc.pack_kv(k, v, P, S)
        frames.append(f)
        orc.scatter_paged(f, t, P, S, H, D, want_k, want_v)
    dk, dv = to_dev(ck), to_dev(cv)
    reqs = [(to_dev(f), torch.from_numpy(t).to(cuda), P) for f, t, P in zip(frames, tables, Ps)]
    scatter_paged_batch(reqs, S, dk, dv)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(to_host(dk), want_k)
    np.testing.assert_array_equal(to_host(dv), want_v)
    for f, t, P in zip(frames, tables, Ps):
        back = gather_paged(dk, dv, t, P, S)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(to_host(back), f)
        np.testing.assert_array_equal(to_host(back), orc.gather_paged(want_k, want_v, t, P, S))


def _attn_case(rng, B, Hq, H, ctx, D=128):
    max_blocks = max((c + 15) // 16 for c in ctx)
    nb = B * max_blocks + 3
    perm = rng.permutation(nb).astype(np.int32)
    tables = np.full((B, max_blocks), -1, np.int32)
    off = 0
    for b, c in enumerate(ctx):
        n = (c + 15) // 16
        tables[b, :n] = perm[off:off + n]
        off += n
    ck = rand_bf16(rng, (nb, H, 16, D))
    cv = rand_bf16(rng, (nb, H, D, 16))
    q = rand_bf16(rng, (B, Hq, D))
    return q, ck, cv, tables, np.asarray(ctx, np.int32)


@pytest.mark.parametrize("B,Hq,H,ctx", [
    (1, 32, 8, [1]),
    (2, 32, 8, [17, 16]),
    (4, 32, 8, [512, 512, 512, 512]),
    (4, 32, 8, [129, 128, 127, 1]),
    (8, 32, 8, [512, 64, 300, 511, 2, 33, 256, 480]),
    (16, 32, 8, [512] * 16),
    (3, 32, 8, [2048, 1500, 700]),
    (2, 8, 8, [200, 37]),
    (2, 16, 8, [200, 37]),
    (2, 64, 8, [200, 37]),
    (2, 128, 8, [300, 5]),
    # KV-head counts that leave a partial group of 8 units, with the query
    # heads of a unit shared by 2 or 4 workgroups
    (1, 12, 3, [200]),
    (3, 6, 3, [100, 517, 33]),
    (2, 24, 3, [700, 1]),
    (5, 80, 5, [64, 1, 999, 300, 16]),
    # a unit's query heads split 8 ways (with the V halves, 16 workgroups per
    # unit) and 16 ways (32 per unit)
    (1, 64, 8, [200]),
    (2, 32, 2, [16, 1]),
    # 128 (stream, KV head) units: one context split up to 2048 tokens (ragged
    # lengths on the whole-context path), then two splits past it
    (16, 32, 8, [2048, 1, 1999, 17, 512, 1024, 2047, 33, 700, 1500, 64, 2000, 129, 900,
                 1800, 5]),
    (16, 32, 8, [3000, 2049, 1, 2048, 100, 2500, 64, 999, 1234, 3000, 7, 2100, 1600, 800,
                 2999, 40]),
])
def test_decode_attention_vs_fp32(cuda, B, Hq, H, ctx):
    from rngd_pd_amd.kernels import decode_attention
    rng = np.random.default_rng(B * 100 + Hq + len(ctx))
    q, ck, cv, tables, ctx_a = _attn_case(rng, B, Hq, H, ctx)
    scale = 1.0 / math.sqrt(128)
    want = orc.decode_attn(q, ck, cv, tables, ctx_a, scale)
    # every output row must be written: start from NaN
    out = torch.full((B, Hq, 128), float("nan"), dtype=torch.bfloat16, device=cuda)
    decode_attention(to_dev(q), to_dev(ck), to_dev(cv), torch.from_numpy(tables).to(cuda),
                     torch.from_numpy(ctx_a).to(cuda), int(ctx_a.max()), scale=scale, out=out)
    torch.cuda.synchronize()
    got = out.float().cpu().numpy()
    np.testing.assert_allclose(got, want, atol=ATOL, rtol=RTOL)


@pytest.mark.parametrize("B,Hq,H,ctx", [(4, 32, 8, [70, 512, 40, 300]), (16, 32, 8, [512] * 16),
                                        (1, 32, 8, [2000]), (3, 32, 2, [100, 600, 17])])
def test_decode_attention_masks_invalid_block_ids(cuda, B, Hq, H, ctx):
    """Block ids outside [0, num_blocks) inside a context mask their tokens, as
    the oracle does: a masked block in the middle, a stream's first two blocks
    (a whole first span, so its running maximum starts at -inf), a stream's
    last partial block, and a stream with every block invalid (zero output);
    one context split and several."""
    from rngd_pd_amd.kernels import decode_attention
    rng = np.random.default_rng(B * 13 + Hq + sum(ctx))
    q, ck, cv, tables, ctx_a = _attn_case(rng, B, Hq, H, ctx)
    nb = ck.shape[0]
    n0 = (ctx[0] + 15) // 16
    tables[0, n0 // 2] = -1
    if B > 1:
        tables[1, :2] = [nb, nb + 100]
    if B > 2:
        tables[2, (ctx[2] - 1) // 16] = -5
    if B > 3:
        tables[3, :(ctx[3] + 15) // 16] = -1
    scale = 1.0 / math.sqrt(128)
    want = orc.decode_attn(q, ck, cv, tables, ctx_a, scale)
    out = torch.full((B, Hq, 128), float("nan"), dtype=torch.bfloat16, device=cuda)
    print(f"attention with invalid block ids B={B} Hq={Hq} H={H} ctx={ctx[:4]}", flush=True)
    decode_attention(to_dev(q), to_dev(ck), to_dev(cv), torch.from_numpy(tables).to(cuda),
                     torch.from_numpy(ctx_a).to(cuda), int(ctx_a.max()), scale=scale, out=out)
    torch.cuda.synchronize()
    got = out.float().cpu().numpy()
    if B > 3:
        assert np.all(got[3] == 0.0)
    np.testing.assert_allclose(got, want, atol=ATOL, rtol=RTOL)


def test_scatter_reports_skipped_block_ids(cuda):
    """Invalid ids in device tables are skipped and counted: the valid blocks
    hold what the oracle's scatter writes (it skips the same ids), nothing
    else changes, and the counter holds one per skipped (request, block)."""
    from rngd_pd_amd.kernels import check_skipped, scatter_paged_batch
    rng = np.random.default_rng(23)
    L, S, H, D = 2, 256, 8, 128
    Ps = [200, 17, 256]
    need = [(p + 15) // 16 for p in Ps]
    nb = sum(need) + 4
    perm = rng.permutation(nb).astype(np.int32)
    tables, off = [], 0
    for n in need:
        tables.append(perm[off:off + n].copy())
        off += n
    tables[0][3] = -1
    tables[0][12] = nb
    tables[2][0] = nb + 9
    ck, cv = _cache(L, nb, H, D)
    want_k, want_v = ck.copy(), cv.copy()
    frames = []
    for P, t in zip(Ps, tables):
        k, v = _prefill(rng, L, S, H, D)
        f = orc.pack_kv(k, v, P, S)
        frames.append(f)
        orc.scatter_paged(f, t, P, S, H, D, want_k, want_v)
    dk, dv = to_dev(ck), to_dev(cv)
    skipped = torch.zeros(1, dtype=torch.int32, device=cuda)
    reqs = [(to_dev(f), torch.from_numpy(t).to(cuda), P) for f, t, P in zip(frames, tables, Ps)]
    print("scatter with invalid block ids", flush=True)
    scatter_paged_batch(reqs, S, dk, dv, skipped=skipped)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(to_host(dk), want_k)
    np.testing.assert_array_equal(to_host(dv), want_v)
    assert int(skipped.item()) == 3
    with pytest.raises(ValueError, match="3 block ids"):
        check_skipped(skipped)
    skipped.zero_()
    scatter_paged_batch(reqs[1:2], S, dk, dv, skipped=skipped)
    check_skipped(skipped)                                    # a valid table: no error


def test_decode_attention_sharing_never_changes_a_result(cuda):
    """At ctx 512 with Hq 32, Hkv 8, batches of 16, 8 and 4 all run one context
    split, but share each (stream, KV head) unit differently: V's dims in two
    halves alone, or also the query heads in 2 or in 4 parts (so 4, 2 or 1
    query heads per wavefront). Streams 0-3 come out bit for bit the same."""
    from rngd_pd_amd.kernels import decode_attention
    rng = np.random.default_rng(31)
    q, ck, cv, tables, ctx_a = _attn_case(rng, 16, 32, 8, [512, 300, 17, 511] * 4)
    dq, dk, dv = to_dev(q), to_dev(ck), to_dev(cv)
    dt, dc = torch.from_numpy(tables).to(cuda), torch.from_numpy(ctx_a).to(cuda)
    outs = []
    for B in (16, 8, 4):
        print(f"sharing: B={B}", flush=True)
        outs.append(decode_attention(dq[:B], dk, dv, dt[:B], dc[:B], 512, scale=0.125))
    torch.cuda.synchronize()
    want = orc.decode_attn(q[:4], ck, cv, tables[:4], ctx_a[:4], 0.125)
    np.testing.assert_allclose(outs[2].float().cpu().numpy(), want, atol=ATOL, rtol=RTOL)
    for o in outs[:2]:
        assert torch.equal(o[:4].view(torch.int16), outs[2].view(torch.int16))


def test_decode_attention_max_ctx_bound_above_actual(cuda):
    """A launch sized for a larger max_ctx gives the same result (empty splits)."""
    from rngd_pd_amd.kernels import decode_attention
    rng = np.random.default_rng(5)
    q, ck, cv, tables, ctx_a = _attn_case(rng, 4, 32, 8, [100, 40, 1, 77])
    tables = np.concatenate([tables, np.full((4, 30), -1, np.int32)], 1)
    want = orc.decode_attn(q, ck, cv, tables, ctx_a, 0.1)
    out = decode_attention(to_dev(q), to_dev(ck), to_dev(cv), torch.from_numpy(tables).to(cuda),
                           torch.from_numpy(ctx_a).to(cuda), 16 * tables.shape[1], scale=0.1)
    torch.cuda.synchronize()
    np.testing.assert_allclose(out.float().cpu().numpy(), want, atol=ATOL, rtol=RTOL)


def test_cache_append_then_attend(cuda):
    from rngd_pd_amd.kernels import cache_append, decode_attention
    rng = np.random.default_rng(9)
    B, Hq, H, D = 4, 32, 8, 128
    q, ck, cv, tables, ctx_a = _attn_case(rng, B, Hq, H, [64, 65, 1, 300])
    k_new = rand_bf16(rng, (B, H, D))
    v_new = rand_bf16(rng, (B, H, D))
    want_k, want_v = ck.copy(), cv.copy()
    orc.cache_append(k_new, v_new, want_k, want_v, tables, ctx_a)
    dk, dv = to_dev(ck), to_dev(cv)
    dt, dc = torch.from_numpy(tables).to(cuda), torch.from_numpy(ctx_a).to(cuda)
    cache_append(to_dev(k_new), to_dev(v_new), dk, dv, dt, dc)
    out = decode_attention(to_dev(q), dk, dv, dt, dc, int(ctx_a.max()), scale=1 / math.sqrt(D))
    torch.cuda.synchronize()
    np.testing.assert_array_equal(to_host(dk), want_k)
    np.testing.assert_array_equal(to_host(dv), want_v)
    want = orc.decode_attn(q, want_k, want_v, tables, ctx_a, 1 / math.sqrt(D))
    np.testing.assert_allclose(out.float().cpu().numpy(), want, atol=ATOL, rtol=RTOL)


@pytest.mark.parametrize("B,V,ld", [(16, 128256, 128256), (3, 1001, 1001), (2, 1000, 1024),
                                    (1, 8, 8)])
def test_greedy_argmax(cuda, B, V, ld):
    """16-byte vector path (aligned rows, V % 8 == 0) and the scalar path."""
    from rngd_pd_amd.kernels import greedy_argmax
    rng = np.random.default_rng(2 + V)
    full = rand_bf16(rng, (B, ld), scale=3.0)
    x = full[:, :V]
    x[0, V - 1] = 0x4380                  # 256.0 in the last column
    if B > 3:
        x[3, V - 2] = x[3, 5] = 0x4400    # a tie (512.0): the first index wins
    if B > 5:
        x[5, 900] = 0x7FC0                # NaN ranks first, and the first NaN wins
        x[5, 77] = 0xFFC1
    want = orc.greedy_argmax(np.ascontiguousarray(x))
    got = greedy_argmax(to_dev(full)[:, :V]).cpu().numpy()
    np.testing.assert_array_equal(got, want)
    assert want[0] == V - 1
    if B > 5:
        assert want[3] == 5 and want[5] == 77


def test_pack_narrow_leaves_tail(cuda):
    """PDK_PACK_NARROW writes K in whole 64-token tiles (zeros past P) and V rows < P,
    and nothing past them."""
    from rngd_pd_amd.kernels import pack_kv_batch, frame_shape
    rng = np.random.default_rng(21)
    L, H, D, S, P = 2, 8, 128, 128, 37
    k, v = _prefill(rng, L, S, H, D)
    full = orc.pack_kv(k, v, P, S)
    frame = torch.full(frame_shape(L, H, D, S), 3.0, dtype=torch.bfloat16, device=cuda)
    pack_kv_batch([(to_dev(k), to_dev(v), P, frame)], S, narrow=True)
    torch.cuda.synchronize()
    got = to_host(frame).reshape(L, 2, -1)
    kf = got[:, 0].reshape(L, H, D, S)
    vf = got[:, 1].reshape(L, H, S, D)
    wk = full.reshape(L, 2, -1)[:, 0].reshape(L, H, D, S)
    wv = full.reshape(L, 2, -1)[:, 1].reshape(L, H, S, D)
    group_end = min((P + 63) // 64 * 64, S)
    np.testing.assert_array_equal(kf[..., :group_end], wk[..., :group_end])
    np.testing.assert_array_equal(vf[:, :, :P], wv[:, :, :P])
    three = np.uint16(0x4040)
    assert (kf[..., group_end:] == three).all() and (vf[:, :, P:] == three).all()


def test_pack_batch_mixing_narrow_and_full_frames(cuda):
    """One launch with a narrow request between two full-width ones (flags per
    request through the C ABI): the full frames equal the oracle's, the narrow one
    holds its valid columns and nothing past them."""
    from rngd_pd_amd import _lib
    from rngd_pd_amd._lib import PackReq
    from rngd_pd_amd.kernels import frame_shape
    rng = np.random.default_rng(23)
    L, H, D, S = 2, 8, 128, 256
    lengths, flags = [200, 37, 256], [0, _lib.PDK_PACK_NARROW, 0]
    srcs = [_prefill(rng, L, S, H, D) for _ in lengths]
    dev = [(to_dev(k), to_dev(v)) for k, v in srcs]
    frames = [torch.full(frame_shape(L, H, D, S), 3.0, dtype=torch.bfloat16, device=cuda)
              for _ in lengths]
    reqs = (PackReq * 3)(*[PackReq(k.data_ptr(), v.data_ptr(), f.data_ptr(), k.stride(0),
                                   k.stride(1), P, fl)
                           for (k, v), f, P, fl in zip(dev, frames, lengths, flags)])
    print(f"pack mixed batch lengths={lengths} flags={flags}", flush=True)
    _lib.call("pdk_pack_kv_batch", reqs, 3, L, S, H, D,
              torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    for (k, v), f, P, fl in zip(srcs, frames, lengths, flags):
        want = orc.pack_kv(k, v, P, S)
        got = to_host(f)
        if not fl:
            np.testing.assert_array_equal(got, want.reshape(got.shape))
            continue
        kf, vf = got.reshape(L, 2, -1)[:, 0].reshape(L, H, D, S), got.reshape(L, 2, -1)[:, 1].reshape(L, H, S, D)
        wk = want.reshape(L, 2, -1)[:, 0].reshape(L, H, D, S)
        wv = want.reshape(L, 2, -1)[:, 1].reshape(L, H, S, D)
        group_end = min((P + 63) // 64 * 64, S)
        np.testing.assert_array_equal(kf[..., :group_end], wk[..., :group_end])
        np.testing.assert_array_equal(vf[:, :, :P], wv[:, :, :P])
        assert (kf[..., group_end:] == np.uint16(0x4040)).all()
        assert (vf[:, :, P:] == np.uint16(0x4040)).all()


def test_decode_attention_workspace_reuse(cuda):
    """Split counters reset themselves: back-to-back calls of different shapes on one
    workspace all match the oracle."""
    from rngd_pd_amd.kernels import decode_attention, get_workspace, workspace_bytes
    rng = np.random.default_rng(31)
    ws = get_workspace(workspace_bytes(16, 32, 2048), cuda)
    for B, ctx in [(16, [512] * 16), (4, [2048, 33, 1000, 512]), (16, [300] * 16), (1, [5])]:
        q, ck, cv, tables, ctx_a = _attn_case(rng, B, 32, 8, ctx)
        want = orc.decode_attn(q, ck, cv, tables, ctx_a, 0.088)
        for _ in range(2):
            out = decode_attention(to_dev(q), to_dev(ck), to_dev(cv),
                                   torch.from_numpy(tables).to(cuda),
                                   torch.from_numpy(ctx_a).to(cuda), int(ctx_a.max()),
                                   scale=0.088, workspace=ws)
            torch.cuda.synchronize()
            np.testing.assert_allclose(out.float().cpu().numpy(), want, atol=ATOL, rtol=RTOL)


def test_decode_attention_graph_replays(cuda):
    """Captured in a HIP graph, every replay (with eager work between replays) equals
    the eager result."""
    from rngd_pd_amd.kernels import decode_attention
    rng = np.random.default_rng(41)
    B = 8
    q, ck, cv, tables, ctx_a = _attn_case(rng, B, 32, 8, [512, 100, 7, 300, 512, 64, 65, 200])
    dq, dk, dv = to_dev(q), to_dev(ck), to_dev(cv)
    dt, dc = torch.from_numpy(tables).to(cuda), torch.from_numpy(ctx_a).to(cuda)
    out = torch.empty_like(dq)
    decode_attention(dq, dk, dv, dt, dc, 512, scale=0.1, out=out)
    torch.cuda.synchronize()
    eager = out.clone()
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            decode_attention(dq, dk, dv, dt, dc, 512, scale=0.1, out=out)
    torch.cuda.synchronize()
    for i in range(4):
        out.zero_()
        decode_attention(dq, dk, dv, dt, dc, 512, scale=0.1, out=torch.empty_like(dq))
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), eager.view(torch.int16)), f"replay {i} differs"


def test_streaming_launches_match_cached_launches(cuda):
    """Launches that move more than 256 MiB use streaming loads/stores; smaller
    ones do not. At full Llama-3.1-8B size, a 4-request batched pack and scatter
    (512 MiB each, streaming) must equal the same requests launched one at a
    time (128 MiB each, ordinary accesses, oracle-checked at small sizes
    above), and a 2048-token gather (512 MiB, streaming) the oracle."""
    from rngd_pd_amd.kernels import (gather_paged, pack_kv, pack_kv_batch, scatter_paged,
                                     scatter_paged_batch)
    L, S, H, D, n = 32, 512, 8, 128, 4
    gen = torch.Generator(device=cuda).manual_seed(21)
    pre = [torch.randn((L, S, 2, H, D), generator=gen, device=cuda).to(torch.bfloat16)
           for _ in range(n)]
    Ps = [512, 509, 497, 512]
    one = [pack_kv(p[:, :, 0], p[:, :, 1], P, S) for p, P in zip(pre, Ps)]
    many = [torch.empty_like(f) for f in one]
    pack_kv_batch([(p[:, :, 0], p[:, :, 1], P, f) for p, P, f in zip(pre, Ps, many)], S)
    torch.cuda.synchronize()
    for a, b in zip(one, many):
        assert torch.equal(a.view(torch.int16), b.view(torch.int16))
    nb = n * (S // 16) + 3
    perm = torch.from_numpy(np.random.default_rng(21).permutation(nb).astype(np.int32)).to(cuda)
    tables = [perm[i * (S // 16):(i + 1) * (S // 16)] for i in range(n)]
    ck1 = torch.zeros((L, nb, H, 16, D), dtype=torch.bfloat16, device=cuda)
    cv1 = torch.zeros((L, nb, H, D, 16), dtype=torch.bfloat16, device=cuda)
    ck2, cv2 = ck1.clone(), cv1.clone()
    for f, t, P in zip(one, tables, Ps):
        scatter_paged(f, t, P, S, ck1, cv1)
    scatter_paged_batch(list(zip(one, tables, Ps)), S, ck2, cv2)
    torch.cuda.synchronize()
    assert torch.equal(ck1.view(torch.int16), ck2.view(torch.int16))
    assert torch.equal(cv1.view(torch.int16), cv2.view(torch.int16))
    del pre, many, ck1, cv1
    # 2048 tokens: one gather moves 512 MiB.
    S2 = 2048
    nb2 = S2 // 16 + 1
    t2 = np.random.default_rng(22).permutation(nb2)[:S2 // 16].astype(np.int32)
    ck = rand_bf16(np.random.default_rng(23), (L, nb2, H, 16, D))
    cv = rand_bf16(np.random.default_rng(24), (L, nb2, H, D, 16))
    got = gather_paged(to_dev(ck), to_dev(cv), torch.from_numpy(t2).to(cuda), 2000, S2)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(to_host(got), orc.gather_paged(ck, cv, t2, 2000, S2))


@pytest.mark.parametrize("blocks", [0, 7])
@pytest.mark.parametrize("nontemporal", [False, True])
def test_stream_probe_moves_every_vector(cuda, blocks, nontemporal):
    """The streaming probes behind the HBM ceilings: a copy reproduces its
    source and a write sets every word, one-shot and grid-stride, including a
    size that is not a whole number of 4 KiB workgroups."""
    from rngd_pd_amd.kernels import stream_probe
    n = (1 << 20) + 48
    src = torch.randint(0, 256, (n,), dtype=torch.uint8, device="cuda")
    dst = torch.zeros(n + 16, dtype=torch.uint8, device="cuda")
    stream_probe("copy", dst=dst, src=src, nbytes=n, nontemporal=nontemporal, blocks=blocks)
    torch.cuda.synchronize()
    assert torch.equal(dst[:n], src)
    assert int(dst[n:].sum()) == 0
    key = 0x01020304
    stream_probe("write", dst=dst, nbytes=n, nontemporal=nontemporal, blocks=blocks, key=key)
    stream_probe("read", src=src, nbytes=n, nontemporal=nontemporal, blocks=blocks)
    torch.cuda.synchronize()
    words = dst[:n].view(torch.int32)
    assert bool((words == key).all())
    assert int(dst[n:].sum()) == 0


@pytest.mark.gpu
def test_attn_read_probe_runs_every_plan(cuda):
    """The loads-only probe launches what decode attention launches (splits,
    shared query heads, partial unit groups) without touching anything but out."""
    from rngd_pd_amd.kernels import attn_read_probe
    rng = np.random.default_rng(7)
    for B, Hq, H, ctx in [(16, 32, 8, [512] * 16), (4, 32, 8, [512, 1, 300, 17]),
                          (3, 12, 3, [2048, 5, 700]), (1, 8, 8, [1])]:
        q, ck, cv, tables, ctx_a = _attn_case(rng, B, Hq, H, ctx)
        dk, dv = to_dev(ck), to_dev(cv)
        out = torch.empty((B, Hq, 128), dtype=torch.bfloat16, device=cuda)
        attn_read_probe(dk, dv, torch.from_numpy(tables).to(cuda), torch.from_numpy(ctx_a).to(cuda),
                        int(ctx_a.max()), Hq, out)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(to_host(dk), ck)
        np.testing.assert_array_equal(to_host(dv), cv)
