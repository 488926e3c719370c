"""decode_batch attention on handed-off KV: prefill KV -> pack -> scatter ->
per-layer decode steps, against the literal restatement of cpu_layer's attention
(oracle.attention.cpu_attention: fp32 einsum, -1e4 mask, new token at pos) on
the reference's dense layout. bf16 outputs within 2e-2 abs / 1e-2 rel."""
import math

import numpy as np
import pytest
import torch

from oracle import attention as oatt
from oracle import native as orc
from tests._util import rand_bf16, to_dev

pytestmark = pytest.mark.gpu

ATOL, RTOL = 2e-2, 1e-2


def _widen(u):
    return (u.astype(np.uint32) << 16).view(np.float32)


@pytest.mark.parametrize("B,lengths,steps", [(4, [512, 512, 512, 512], 2),
                                             (3, [100, 37, 300], 3),
                                             (16, [512] * 16, 1)])
def test_decode_steps_on_handed_off_kv(cuda, B, lengths, steps):
    from rngd_pd_amd import kernels as K
    from rngd_pd_amd.engines.decode_batch import BatchDecodeAttention
    from rngd_pd_amd.engines.paged_cache import PagedKVCache
    L, H, D, Hq = 2, 8, 128, 32
    S = 512 + 16 * steps
    rng = np.random.default_rng(B + steps)
    cache = PagedKVCache(L, B * (S // 16 + 1), H, D, device=cuda, seed=B)
    eng = BatchDecodeAttention(cache, n_q_heads=Hq)
    dense_k = np.zeros((L, B, H, D, S), np.float32)
    dense_v = np.zeros((L, B, H, S, D), np.float32)
    ids = [f"s{b}" for b in range(B)]
    for b, P in enumerate(lengths):
        k, v = rand_bf16(rng, (L, P, H, D)), rand_bf16(rng, (L, P, H, D))
        frame = K.pack_kv(to_dev(k), to_dev(v), P, S)
        eng.admit(ids[b], frame, P, S)
        dense_k[:, b, :, :, :P] = np.transpose(_widen(k), (0, 2, 3, 1))
        dense_v[:, b, :, :P, :] = np.transpose(_widen(v), (0, 2, 1, 3))
    for step in range(steps):
        tables, ctx, max_ctx = eng.prepare(ids)
        positions = [eng.positions[r] for r in ids]
        for layer in range(L):
            q = rand_bf16(rng, (B, Hq, D))
            kn, vn = rand_bf16(rng, (B, H, D)), rand_bf16(rng, (B, H, D))
            out = eng.layer_attention(layer, to_dev(q), to_dev(kn), to_dev(vn), tables, ctx, max_ctx)
            torch.cuda.synchronize()
            want = oatt.cpu_attention(_widen(q), dense_k[layer], dense_v[layer], positions,
                                      _widen(kn), _widen(vn))
            np.testing.assert_allclose(out.float().cpu().numpy(), want, atol=ATOL, rtol=RTOL)
            for b, p in enumerate(positions):          # keep the dense reference in step
                dense_k[layer, b, :, :, p] = _widen(kn[b])
                dense_v[layer, b, :, p, :] = _widen(vn[b])
        eng.advance(ids)
    eng.retire(ids[0])
    assert ids[0] not in cache._tables


def test_full_llama_shape_all_layers(cuda):
    """Config-3 shape: B=16, 32 query / 8 KV heads, ctx 512, 32 layers, vs the C oracle."""
    from rngd_pd_amd import kernels as K
    L, B, H, Hq, D, ctx = 32, 16, 8, 32, 128, 512
    gen = torch.Generator(device=cuda).manual_seed(0)
    nb = B * ctx // 16
    ck = torch.randn((L, nb, H, 16, D), generator=gen, device=cuda).to(torch.bfloat16)
    cv = torch.randn((L, nb, H, D, 16), generator=gen, device=cuda).to(torch.bfloat16)
    q = torch.randn((L, B, Hq, D), generator=gen, device=cuda).to(torch.bfloat16)
    tables = torch.from_numpy(np.random.default_rng(0).permutation(nb).astype(np.int32)
                              .reshape(B, -1)).to(cuda)
    ctx_t = torch.full((B,), ctx, dtype=torch.int32, device=cuda)
    outs = [K.decode_attention(q[l], ck[l], cv[l], tables, ctx_t, ctx, scale=1 / math.sqrt(D))
            for l in range(L)]
    torch.cuda.synchronize()
    h = lambda t: t.cpu().contiguous().view(torch.int16).numpy().view(np.uint16)   # noqa: E731
    for l in (0, 13, 31):
        want = orc.decode_attn(h(q[l]), h(ck[l]), h(cv[l]), tables.cpu().numpy(),
                               ctx_t.cpu().numpy(), 1 / math.sqrt(D))
        np.testing.assert_allclose(outs[l].float().cpu().numpy(), want, atol=ATOL, rtol=RTOL)
