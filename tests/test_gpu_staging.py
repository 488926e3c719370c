"""The handoff staged through pinned host memory, against the oracle.

The batch is the GPU handoff workload: 8 Llama-3.1-8B requests (32 layers,
8 KV heads, head_dim 128, S=512 frames) with lengths uniform in [64, 512] from
seed 0, a paged cache of block size 16 with a seeded permuted block table.
Both staging modes must leave (a) every request's pinned host frame equal to
the oracle's S-wide frame (the wire payloads, zero tail included) and (b) the
paged cache equal to the oracle's scatter of those frames, bit for bit. A
second batch of other lengths through the same pinned slots checks that a
shorter request rewrites the zero tail a longer one left dirty.
"""
import numpy as np
import pytest
import torch

from oracle import native as orc
from tests._util import to_dev, to_host

pytestmark = pytest.mark.gpu

L, H, D, S = 32, 8, 128, 512


def _lengths(seed, n=8):
    return [int(p) for p in np.random.default_rng(seed).integers(64, S + 1, n)]


def _batch(rng, lengths, nb, cuda):
    """Random bf16 bit patterns (every bit pattern, NaNs included: the path only
    moves bits) and a permuted block table per request."""
    perm = rng.permutation(nb).astype(np.int32)
    reqs, off = [], 0
    for P in lengths:
        kv = rng.integers(0, 1 << 16, (L, 2, S, H, D), dtype=np.uint16)
        n = (P + 15) // 16
        reqs.append((kv, perm[off:off + n].copy(), P))
        off += n
    return reqs


def _run_and_check(stager, reqs, nb, cuda, fill):
    ck = np.full((L, nb, H, 16, D), fill, np.uint16)
    cv = np.full((L, nb, H, D, 16), fill, np.uint16)
    want_k, want_v = ck.copy(), cv.copy()
    frames = []
    for kv, table, P in reqs:
        f = orc.pack_kv(kv[:, 0], kv[:, 1], P, S)
        orc.scatter_paged(f, table, P, S, H, D, want_k, want_v)
        frames.append(f)
    dk, dv = to_dev(ck, cuda), to_dev(cv, cuda)
    dev_kv = [to_dev(kv, cuda) for kv, _, _ in reqs]
    args = [(d[:, 0], d[:, 1], P, torch.from_numpy(t).to(cuda))
            for d, (_, t, P) in zip(dev_kv, reqs)]
    stager.run(args, dk, dv)
    torch.cuda.synchronize()
    for r, f in enumerate(frames):
        np.testing.assert_array_equal(stager.host_frame(r), f, err_msg=f"host frame {r}")
    np.testing.assert_array_equal(to_host(dk), want_k)
    np.testing.assert_array_equal(to_host(dv), want_v)


@pytest.mark.parametrize("mode", ["kernel", "dma"])
def test_staged_batch_matches_oracle(cuda, mode):
    from rngd_pd_amd.kernels.staging import HostStagedHandoff
    first, second = _lengths(0), _lengths(7)
    nb = max(sum((p + 15) // 16 for p in ls) for ls in (first, second)) + 16
    stager = HostStagedHandoff(L, H, D, S, 8, device=cuda, mode=mode)
    try:
        rng = np.random.default_rng(21)
        print(f"staged {mode}: lengths {first}", flush=True)
        _run_and_check(stager, _batch(rng, first, nb, cuda), nb, cuda, fill=0)
        # Same slots, other lengths: tails a longer request left must be zero again.
        print(f"staged {mode}: lengths {second}", flush=True)
        _run_and_check(stager, _batch(rng, second, nb, cuda), nb, cuda, fill=0x3F80)
    finally:
        stager.close()


@pytest.mark.parametrize("mode,copy_bytes", [("kernel", None), ("dma", 16 << 20),
                                             ("dma", 1 << 20)])
def test_staged_edge_lengths(cuda, mode, copy_bytes):
    """P = 0 (nothing to place, frame all zero), 1, 16, 17 and S in one batch;
    "dma" mode also with copies of about 1 MiB (several per request)."""
    from rngd_pd_amd.kernels.staging import HostStagedHandoff
    lengths = [0, 1, 16, 17, S]
    nb = sum((p + 15) // 16 for p in lengths) + 4
    kw = {} if copy_bytes is None else {"copy_bytes": copy_bytes}
    stager = HostStagedHandoff(L, H, D, S, len(lengths), device=cuda, mode=mode, **kw)
    if mode == "dma":
        # A full-length request has 2 MiB of valid columns per layer.
        per_copy = max(1, min(L, copy_bytes // (2 * S * H * D * 2)))
        chunks = stager.layer_chunks(S)
        assert [l0 for l0, _ in chunks] == list(range(0, L, per_copy))
        assert sum(n for _, n in chunks) == L
    try:
        reqs = _batch(np.random.default_rng(5), lengths, nb, cuda)
        reqs[0] = (reqs[0][0], np.zeros(1, np.int32), 0)
        _run_and_check(stager, reqs, nb, cuda, fill=0x1234)
    finally:
        stager.close()


def test_staged_rejects_bad_input(cuda):
    from rngd_pd_amd.kernels.staging import HostStagedHandoff
    stager = HostStagedHandoff(2, H, D, 64, 2, device=cuda)
    try:
        kv = torch.zeros((2, 2, 64, H, D), dtype=torch.bfloat16, device=cuda)
        ck = torch.zeros((2, 8, H, 16, D), dtype=torch.bfloat16, device=cuda)
        cv = torch.zeros((2, 8, H, D, 16), dtype=torch.bfloat16, device=cuda)
        short = torch.zeros(1, dtype=torch.int32, device=cuda)
        with pytest.raises(ValueError, match="block table"):
            stager.run([(kv[:, 0], kv[:, 1], 40, short)], ck, cv)
        with pytest.raises(ValueError, match="num_tokens"):
            stager.run([(kv[:, 0], kv[:, 1], 65, short)], ck, cv)
        with pytest.raises(ValueError, match="requests per run"):
            stager.run([(kv[:, 0], kv[:, 1], 1, short)] * 3, ck, cv)
    finally:
        stager.close()


def test_copy_frame_valid_parts(cuda):
    """pdk_copy_frame_valid copies exactly the requested parts: K rows' first
    min(round16(P), S) columns and V rows < P, for a range of layers, each way;
    every other byte of the destination keeps what it held."""
    import ctypes
    from rngd_pd_amd import _lib
    from rngd_pd_amd.hip import PinnedBuffer
    lib = _lib.lib()
    Lf, Hf, Df, Sf = 5, 2, 64, 144
    F = Hf * Df * Sf
    rng = np.random.default_rng(11)
    src = rng.integers(0, 1 << 16, (Lf, 2, F), dtype=np.uint16)
    dframe = to_dev(src, cuda)
    pin = PinnedBuffer(Lf * 2 * F * 2)
    host = pin.view(np.uint16, 0, Lf * 2 * F).reshape(Lf, 2, F)
    st = torch.cuda.current_stream(cuda).cuda_stream
    for P in (1, 15, 16, 17, 100, 129, Sf):
        k1 = min((P + 15) // 16 * 16, Sf)
        for parts in (_lib.PDK_FRAME_K, _lib.PDK_FRAME_V, _lib.PDK_FRAME_KV):
            l0, nl = 1, 3
            host[:] = 0xBEEF
            rc = lib.pdk_copy_frame_valid(ctypes.c_void_p(pin.ptr), ctypes.c_void_p(dframe.data_ptr()),
                                          l0, nl, Hf, Df, Sf, P, _lib.PDK_COPY_D2H, parts, st)
            assert rc == 0, _lib.last_error()
            torch.cuda.synchronize()
            copied = np.zeros(src.shape, bool)
            if parts & _lib.PDK_FRAME_K:
                copied[:, 0].reshape(Lf, Hf * Df, Sf)[l0:l0 + nl, :, :k1] = True
            if parts & _lib.PDK_FRAME_V:
                copied[:, 1].reshape(Lf, Hf, Sf, Df)[l0:l0 + nl, :, :P] = True
            want = np.where(copied, src, np.uint16(0xBEEF))
            np.testing.assert_array_equal(host, want, err_msg=f"down P={P} parts={parts}")
            # And back up into a device frame holding a pattern.
            back = to_dev(np.full_like(src, 0x1234), cuda)
            host[:] = src
            rc = lib.pdk_copy_frame_valid(ctypes.c_void_p(back.data_ptr()), ctypes.c_void_p(pin.ptr),
                                          l0, nl, Hf, Df, Sf, P, _lib.PDK_COPY_H2D, parts, st)
            assert rc == 0, _lib.last_error()
            torch.cuda.synchronize()
            want = np.where(copied, src, np.uint16(0x1234))
            np.testing.assert_array_equal(to_host(back), want, err_msg=f"up P={P} parts={parts}")
    for bad in (0, 4):
        assert lib.pdk_copy_frame_valid(ctypes.c_void_p(pin.ptr), ctypes.c_void_p(dframe.data_ptr()),
                                        0, 1, Hf, Df, Sf, 16, _lib.PDK_COPY_D2H, bad, st) \
            == _lib.PDK_EINVAL
    torch.cuda.synchronize()
    pin.close()
