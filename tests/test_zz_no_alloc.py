"""pdk_decode_attn_noalloc (split partials in the library's own device array)
against pdk_decode_attn with a caller workspace, through the C ABI.

Shapes are chosen so that the launch splits the context (partials in the
scratch array): the outputs must be bit-identical, on two calls in a row, the
second with a smaller input (fewer streams, shorter contexts), and a launch
that would need more scratch than the array holds is refused.
"""
import ctypes
import math

import numpy as np
import pytest
import torch

from tests._util import rand_bf16, to_dev

pytestmark = pytest.mark.gpu


def _case(rng, B, Hq, H, ctx, D=128):
    max_blocks = max((c + 15) // 16 for c in ctx)
    nb = B * max_blocks + 3
    perm = rng.permutation(nb).astype(np.int32)
    tables = np.full((B, max_blocks), -1, np.int32)
    off = 0
    for b, c in enumerate(ctx):
        n = (c + 15) // 16
        tables[b, :n] = perm[off:off + n]
        off += n
    return (rand_bf16(rng, (B, Hq, D)), rand_bf16(rng, (nb, H, 16, D)),
            rand_bf16(rng, (nb, H, D, 16)), tables, np.asarray(ctx, np.int32))


def _both(lib, cuda, q, ck, cv, tables, ctx, Hq, H):
    B = q.shape[0]
    D = q.shape[2]
    nb = ck.shape[0]
    max_ctx = int(ctx.max())
    dq, dk, dv = to_dev(q, cuda), to_dev(ck, cuda), to_dev(cv, cuda)
    dt, dc = torch.from_numpy(tables).to(cuda), torch.from_numpy(ctx).to(cuda)
    scale = 1.0 / math.sqrt(D)
    st = torch.cuda.current_stream().cuda_stream
    wsb = lib.pdk_decode_attn_workspace_bytes(B, Hq, max_ctx, D)
    assert wsb > 0, "the case must split the context"
    ws = torch.empty(wsb, dtype=torch.uint8, device=cuda)
    want = torch.empty((B, Hq, D), dtype=torch.bfloat16, device=cuda)
    got = torch.full((B, Hq, D), 7.0, dtype=torch.bfloat16, device=cuda)
    rc = lib.pdk_decode_attn(dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), nb, dt.data_ptr(),
                             tables.shape[1], dc.data_ptr(), max_ctx, B, Hq, H, D, scale,
                             ws.data_ptr(), wsb, want.data_ptr(), st)
    assert rc == 0, lib.pdk_last_error().decode()
    rc = lib.pdk_decode_attn_noalloc(dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), nb,
                                     dt.data_ptr(), tables.shape[1], dc.data_ptr(), max_ctx, B,
                                     Hq, H, D, scale, got.data_ptr(), st)
    assert rc == 0, lib.pdk_last_error().decode()
    torch.cuda.synchronize()
    return got, want


def test_noalloc_matches_workspace_entry_point(cuda):
    from rngd_pd_amd import _lib
    lib = _lib.lib()
    rng = np.random.default_rng(31)
    cases = [(4, 32, 8, [2048, 1500, 700, 33]),      # first call: 4 splits of 512 tokens
             (2, 32, 8, [600, 129])]                   # second, smaller: 5 splits of 128
    for B, Hq, H, ctx in cases:
        print(f"noalloc vs workspace: B={B} Hq={Hq} Hkv={H} ctx={ctx}", flush=True)
        q, ck, cv, tables, ctx_a = _case(rng, B, Hq, H, ctx)
        got, want = _both(lib, cuda, q, ck, cv, tables, ctx_a, Hq, H)
        assert torch.equal(got.view(torch.int16), want.view(torch.int16))


def test_noalloc_refuses_more_than_its_scratch(cuda):
    """255 streams of one KV head with 16 query heads at context 4096 split in two:
    4.2 MB of partials, more than the array holds. Refused before any launch.
    Every buffer is sized for the call (one cache block, every table entry 0), so
    the call would stay in bounds even if a later launch plan did not refuse it."""
    from rngd_pd_amd import _lib
    lib = _lib.lib()
    B, Hq, H, D, max_ctx = 255, 16, 1, 128, 4096
    max_blocks = max_ctx // 16
    q = torch.zeros((B, Hq, D), dtype=torch.bfloat16, device=cuda)
    ck = torch.zeros((1, H, 16, D), dtype=torch.bfloat16, device=cuda)
    cv = torch.zeros((1, H, D, 16), dtype=torch.bfloat16, device=cuda)
    tables = torch.zeros((B, max_blocks), dtype=torch.int32, device=cuda)
    ctx = torch.full((B,), max_ctx, dtype=torch.int32, device=cuda)
    out = torch.zeros((B, Hq, D), dtype=torch.bfloat16, device=cuda)
    need = B * Hq * 2 * (D + 2) * 4                      # partials of two splits
    assert need > 4 << 20                                # PDK_NOALLOC_SCRATCH_BYTES
    rc = lib.pdk_decode_attn_noalloc(q.data_ptr(), ck.data_ptr(), cv.data_ptr(), 1,
                                     tables.data_ptr(), max_blocks, ctx.data_ptr(), max_ctx,
                                     B, Hq, H, D, 0.1, out.data_ptr(),
                                     torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert rc == _lib.PDK_ENOMEM, (rc, lib.pdk_last_error())
    assert b"no-allocation" in lib.pdk_last_error()
