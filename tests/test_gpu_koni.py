"""KONI token blocks into the paged cache on the GPU (pdk_scatter_koni through
KoniPagedReceiver), against the oracle receiver (oracle/koni.py, the
reference's KVReceiver restated): every placed value bit for bit, and every
slot the request does not own (or has not received) untouched."""
import numpy as np
import pytest
import torch

from oracle import attention as oatt
from oracle import koni as ok
from tests._util import to_host

pytestmark = pytest.mark.gpu

L, H, D = 32, 8, 128


def _runs(rng, t, n):
    """Split tokens 0..n-1 of tensor t into random runs -> entries."""
    out, tok = [], 0
    while tok < n:
        c = int(rng.integers(1, min(6, n - tok) + 1))
        out.append(dict(tier=0, tensor=t, block=tok, bytes=c * 2048))
        tok += c
    return out


@pytest.mark.parametrize("n", [1, 17, 300])
def test_koni_batches_into_paged_cache(cuda, n):
    from rngd_pd_amd.connector import koni
    from rngd_pd_amd.engines.paged_cache import PagedKVCache
    rng = np.random.default_rng(n)
    nb = (n + 15) // 16 + 5
    cache = PagedKVCache(L, nb, H, D, device=cuda, seed=n)
    g = torch.Generator(device=cuda).manual_seed(n)
    cache.k.copy_(torch.randn(cache.k.shape, generator=g, device=cuda))
    cache.v.copy_(torch.randn(cache.v.shape, generator=g, device=cuda))
    k0, v0 = to_host(cache.k), to_host(cache.v)
    view = cache.view("r", n, (n + 15) // 16 * 16)
    bits = rng.integers(0, 65536, size=(2 * L, n, H, D), dtype=np.uint16)
    bits &= 0x7FFF                                     # no NaN patterns (any bits are carried)
    entries = [e for t in range(2 * L) for e in _runs(rng, t, n)]
    order = rng.permutation(len(entries))
    entries = [entries[i] for i in order]
    cut = len(entries) // 2
    recv = koni.KoniPagedReceiver("r", n, view)
    orc = ok.Receiver("r", n)
    print(f"koni n={n}: {len(entries)} entries in 2 batches", flush=True)
    for batch, final in ((entries[:cut], False), (entries[cut:], True)):
        if not batch:
            continue
        raw = b"".join(bits[e["tensor"], e["block"]:e["block"] + e["bytes"] // 2048]
                       .astype("<u2").tobytes() for e in batch)
        cuts = sorted(set([0, len(raw)] + rng.integers(0, len(raw), size=9).tolist()))
        frames = [raw[a:b] for a, b in zip(cuts, cuts[1:])]
        msg = koni.parse(koni.kv_message("r", batch, final))
        assert orc.accept(msg, frames) == final
        assert recv.accept(msg, frames) == final
    recv.close()
    got_k, got_v = to_host(cache.k), to_host(cache.v)
    blocks = cache.blocks("r")
    want_k, want_v = k0.copy(), v0.copy()
    kbits = (orc.keys.view(np.uint32) >> 16).astype(np.uint16)       # [L, H, D, n]
    vbits = (orc.values.view(np.uint32) >> 16).astype(np.uint16)     # [L, H, n, D]
    rows = oatt.k_block_rows(want_k)                                  # [L, nb, H, 16, D]
    for j, blk in enumerate(blocks):
        m = min(16, n - 16 * j)
        rows[:, blk, :, :m, :] = kbits[:, :, :, 16 * j:16 * j + m].transpose(0, 1, 3, 2)
        want_v[:, blk, :, :, :m] = vbits[:, :, 16 * j:16 * j + m, :].transpose(0, 1, 3, 2)
    want_k = oatt.k_block_tiled(rows)
    np.testing.assert_array_equal(got_k, want_k)
    np.testing.assert_array_equal(got_v, want_v)
