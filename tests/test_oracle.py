"""Pins of the CPU oracle (oracle/), each against something other than itself.

  wire       closed form of the bf16 truncation, torch's bf16 cast on bf16-valued
             data, and the reference's own test vectors (tests/test_airm.py:93-103,
             :166-175: seeds 0 and 1, shapes (8,16,128) and (2,2,4,2,8));
  pack       numpy transposes (independent of the C loops);
  scatter    numpy fancy indexing (oracle.attention.paged_from_dense) and the
             gather round trip;
  attention  torch float64 softmax attention, the literal numpy restatement of
             cpu_layer (fp32 einsum, -1e4 mask), and closed-form special cases;
  argmax     torch.argmax (first maximum; NaN ranks first).
A planted mistake (a transposed operand) is shown to fail the pack pin.
"""
import math
import os

import numpy as np
import pytest
import torch

from oracle import attention as oatt
from oracle import native as orc
from oracle import wire as owire

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _bf16_valued(rng, shape, scale=1.0):
    x = (rng.standard_normal(shape) * scale).astype(np.float32)
    return (x.view(np.uint32) >> 16 << 16).view(np.float32)


def _bits(x):
    return (np.ascontiguousarray(x, np.float32).view(np.uint32) >> 16).astype(np.uint16)


# ---------------------------------------------------------------- wire -----
def test_truncate_is_high_half():
    rng = np.random.default_rng(3)
    x = rng.standard_normal(4096).astype(np.float32) * 100
    got = orc.bf16_truncate(x)
    np.testing.assert_array_equal(got, (x.view(np.uint32) >> 16).astype(np.uint16))
    # truncation, not rounding: differs from round-to-nearest on some inputs
    rne = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert (got != rne).any()


def test_truncate_equals_torch_cast_on_bf16_values():
    x = _bf16_valued(np.random.default_rng(4), (64, 128))
    rne = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    np.testing.assert_array_equal(orc.bf16_truncate(x), rne)
    np.testing.assert_array_equal(orc.bf16_widen(rne), x)


def test_reference_vector_adapter_round_trip():
    """tests/test_airm.py:166-175: seed 1, (2,2,4,2,8), got bits == in bits >> 16 << 16."""
    kv_in = np.random.default_rng(1).standard_normal((2, 2, 4, 2, 8)).astype(np.float32)
    got = owire.deser(owire.ser(kv_in, "bf16")).reshape(kv_in.shape)
    np.testing.assert_array_equal(got.view(np.uint32), kv_in.view(np.uint32) >> 16 << 16)


def test_reference_vector_connector_seed0():
    """tests/test_airm.py:25-28,93-103: _kv(0) layers through the bf16 wire."""
    rng = np.random.default_rng(0)
    ck = [rng.standard_normal((8, 16, 128)).astype(np.float32) for _ in range(4)]
    for a in ck:
        got = owire.deser(owire.ser(a, "bf16"))
        np.testing.assert_array_equal(got, (a.view(np.uint32) >> 16 << 16).view(np.float32))


def test_fp16_wire_loss():
    """connector/transport.py:364-379: fp16 round trip equals astype(float16)."""
    arr = np.random.default_rng(0).standard_normal((8, 16, 128)).astype(np.float32)
    got = owire.deser(owire.ser(arr, "fp16"))
    assert np.abs(got - arr.astype(np.float16).astype(np.float32)).max() < 1e-6


def test_blob_envelope_geometry():
    """A Llama-8B layer frame (8,128,512) pickles to 1,048,769 bytes with the
    payload at byte 161 under numpy 2.x (numpy 1.x names numpy.core: one byte less)."""
    x = _bf16_valued(np.random.default_rng(5), (8, 128, 512))
    blob = owire.ser(x, "bf16")
    payload = _bits(x).tobytes()
    off = blob.find(payload)
    if np.__version__.startswith("2."):
        assert (len(blob), off) == (1048769, 161)
    assert off > 0 and len(blob) - off - len(payload) > 0


def test_shm_protocol_files(tmp_path):
    root = str(tmp_path)
    owire.shm_push(root, "req/layer.0/k", b"abc")
    assert os.listdir(root) == ["req__layer.0__k"]
    assert owire.shm_pull(root, "req/layer.0/k") == b"abc"
    with pytest.raises(TimeoutError):
        owire.shm_pull(root, "req/layer.1/k", timeout=0.01)


def test_golden_blobs():
    """Committed blobs (tests/golden/make_golden.py) still come out byte for byte."""
    z = np.load(os.path.join(GOLDEN, "wire_blobs.npz"))
    for name in ("small", "adapter"):
        x = z[f"{name}_in"]
        assert owire.ser(x, "bf16") == z[f"{name}_blob"].tobytes()


# ---------------------------------------------------------------- pack -----
def _numpy_frame(k, v, P, S):
    """Independent formulation: K -> [L, H, D, S], V -> [L, H, S, D], zero tail."""
    L, T, H, D = k.shape
    K = np.zeros((L, H, D, S), np.uint16)
    V = np.zeros((L, H, S, D), np.uint16)
    K[..., :P] = np.transpose(k[:, :P], (0, 2, 3, 1))
    V[:, :, :P] = np.transpose(v[:, :P], (0, 2, 1, 3))
    return np.stack([K.reshape(L, -1), V.reshape(L, -1)], 1)


@pytest.mark.parametrize("L,T,S,P,H,D", [(2, 16, 16, 16, 8, 128), (3, 40, 48, 33, 2, 64),
                                         (1, 64, 64, 0, 4, 32), (2, 20, 32, 20, 1, 8)])
def test_pack_matches_numpy_transpose(L, T, S, P, H, D):
    rng = np.random.default_rng(P + T)
    k = _bits(_bf16_valued(rng, (L, T, H, D)))
    v = _bits(_bf16_valued(rng, (L, T, H, D)))
    np.testing.assert_array_equal(orc.pack_kv(k, v, P, S), _numpy_frame(k, v, P, S))


def test_pack_equals_reference_frame_builder():
    """The frame equals what the reference's prefill writes per layer: its K/V
    caches ([NKV, HD, S] / [NKV, S, HD], zero past P) as bf16 bits."""
    rng = np.random.default_rng(8)
    L, T, H, D, S, P = 2, 24, 8, 128, 32, 21
    kv = _bf16_valued(rng, (L, 2, T, H, D))
    Kf, Vf = owire.frames_from_prefill(kv, P, S)
    frame = orc.pack_kv(_bits(kv[:, 0]), _bits(kv[:, 1]), P, S)
    for l in range(L):
        assert frame[l, 0].tobytes() == _bits(Kf[l]).tobytes()
        assert frame[l, 1].tobytes() == _bits(Vf[l]).tobytes()


def test_planted_transpose_mistake_is_caught():
    """Swapping the K transpose axes (a plausible slip) fails the pack pin."""
    rng = np.random.default_rng(9)
    L, T, H, D, S, P = 1, 16, 2, 16, 16, 16
    k = _bits(_bf16_valued(rng, (L, T, H, D)))
    v = _bits(_bf16_valued(rng, (L, T, H, D)))
    wrong = _numpy_frame(k, v, P, S)
    wrong[:, 0] = np.transpose(k, (0, 2, 1, 3)).reshape(L, -1)   # [L, H, T, D]: not transposed
    assert not np.array_equal(orc.pack_kv(k, v, P, S), wrong)


# ------------------------------------------------------------- scatter -----
@pytest.mark.parametrize("P", [1, 15, 16, 17, 40, 64])
def test_scatter_matches_numpy_indexing_and_round_trips(P):
    rng = np.random.default_rng(P)
    L, H, D, S = 2, 2, 32, 64
    nb = 9
    k = _bits(_bf16_valued(rng, (L, S, H, D)))
    v = _bits(_bf16_valued(rng, (L, S, H, D)))
    frame = orc.pack_kv(k, v, P, S)
    table = rng.permutation(nb)[:(P + 15) // 16].astype(np.int32)
    ck = np.full((L, nb, H, 16, D), 7, np.uint16)
    cv = np.full((L, nb, H, D, 16), 7, np.uint16)
    orc.scatter_paged(frame, table, P, S, H, D, ck, cv)
    for l in range(L):
        K = frame[l, 0].reshape(1, H, D, S)
        V = frame[l, 1].reshape(1, H, S, D)
        wk, wv = oatt.paged_from_dense(K, V, [P], table[None, :], nb)
        kr, wkr = oatt.k_block_rows(ck[l]), oatt.k_block_rows(wk)   # token rows
        for j, blk in enumerate(table):
            n = min(16, P - 16 * j)
            np.testing.assert_array_equal(kr[blk, :, :n], wkr[blk, :, :n])
            np.testing.assert_array_equal(cv[l, blk, :, :, :n], wv[blk, :, :, :n])
            assert (kr[blk, :, n:] == 0).all() and (cv[l, blk, :, :, n:] == 0).all()
        untouched = sorted(set(range(nb)) - set(table.tolist()))
        assert (ck[l, untouched] == 7).all() and (cv[l, untouched] == 7).all()
    np.testing.assert_array_equal(orc.gather_paged(ck, cv, table, P, S), frame)


# ----------------------------------------------------------- attention -----
def _attn_case(rng, B, Hq, H, ctx, D):
    mb = max((c + 15) // 16 for c in ctx)
    nb = B * mb + 1
    perm = rng.permutation(nb).astype(np.int32)
    tables = np.full((B, mb), -1, np.int32)
    off = 0
    for b, c in enumerate(ctx):
        n = (c + 15) // 16
        tables[b, :n] = perm[off:off + n]
        off += n
    ck = _bits(_bf16_valued(rng, (nb, H, 16, D)))
    cv = _bits(_bf16_valued(rng, (nb, H, D, 16)))
    q = _bits(_bf16_valued(rng, (B, Hq, D)))
    return q, ck, cv, tables, np.asarray(ctx, np.int32)


def _torch_f64_attention(q, ck, cv, tables, ctx, scale):
    """softmax(q k^T * scale) v in float64, each stream's keys gathered by token."""
    B, Hq, D = q.shape
    H = ck.shape[1]
    G = Hq // H
    w = lambda u: torch.from_numpy(orc.bf16_widen(u)).double()   # noqa: E731
    Q, CK, CV = w(q), w(oatt.k_block_rows(ck)), w(cv)             # K as token rows
    out = torch.zeros((B, Hq, D), dtype=torch.float64)
    for b in range(B):
        t = torch.arange(int(ctx[b]))
        blk = torch.from_numpy(tables[b].astype(np.int64))[t // 16]
        Kb = CK[blk, :, t % 16, :]               # [T, H, D]
        Vb = CV[blk, :, :, t % 16]               # [T, H, D]
        for qh in range(Hq):
            s = (Kb[:, qh // G] @ Q[b, qh]) * scale
            out[b, qh] = torch.softmax(s, 0) @ Vb[:, qh // G]
    return out.numpy()


@pytest.mark.parametrize("B,Hq,H,ctx", [(1, 4, 1, [1]), (2, 8, 2, [17, 40]),
                                        (3, 32, 8, [64, 5, 33]), (2, 16, 16, [20, 48])])
def test_attention_matches_torch_float64(B, Hq, H, ctx):
    rng = np.random.default_rng(B * 10 + Hq)
    q, ck, cv, tables, c = _attn_case(rng, B, Hq, H, ctx, 32)
    scale = 1 / math.sqrt(32)
    np.testing.assert_allclose(orc.decode_attn(q, ck, cv, tables, c, scale),
                               _torch_f64_attention(q, ck, cv, tables, c, scale),
                               rtol=1e-5, atol=1e-6)


def test_attention_masks_invalid_block_ids():
    """A block id outside [0, num_blocks) inside the context masks that block's
    tokens: the result is the float64 softmax attention over the other
    tokens alone (gathered by token, the invalid ones dropped), and a stream
    with no valid block gets zeros."""
    rng = np.random.default_rng(14)
    B, Hq, H, D = 3, 8, 2, 32
    q, ck, cv, tables, c = _attn_case(rng, B, Hq, H, [70, 40, 33], D)
    nb = ck.shape[0]
    tables[0, 1] = -1                      # tokens 16..31 of stream 0
    tables[0, 4] = nb + 3                  # its last, partial block
    tables[1, 0] = nb                      # stream 1's first block
    tables[2, :3] = -7                     # every block of stream 2
    scale = 1 / math.sqrt(D)
    got = orc.decode_attn(q, ck, cv, tables, c, scale)
    w = lambda u: torch.from_numpy(orc.bf16_widen(u)).double()   # noqa: E731
    Q, CK, CV = w(q), w(oatt.k_block_rows(ck)), w(cv)
    for b in range(B):
        t = torch.tensor([i for i in range(int(c[b])) if 0 <= tables[b, i // 16] < nb],
                         dtype=torch.int64)
        if t.numel() == 0:
            np.testing.assert_array_equal(got[b], 0.0)
            continue
        blk = torch.from_numpy(tables[b].astype(np.int64))[t // 16]
        Kb, Vb = CK[blk, :, t % 16, :], CV[blk, :, :, t % 16]
        for qh in range(Hq):
            s_ = (Kb[:, qh // (Hq // H)] @ Q[b, qh]) * scale
            want = (torch.softmax(s_, 0) @ Vb[:, qh // (Hq // H)]).numpy()
            np.testing.assert_allclose(got[b, qh], want, rtol=1e-5, atol=1e-6)


def test_attention_matches_cpu_layer_restatement():
    """The literal cpu_layer lines (kernels/decode_batch.py:147-156) on the dense
    layout, including the new-token write at positions[b]."""
    rng = np.random.default_rng(12)
    B, NH, NKV, HD, S = 3, 32, 8, 128, 48
    positions = [5, 47, 20]
    q = _bf16_valued(rng, (B, NH, HD))
    K = _bf16_valued(rng, (B, NKV, HD, S))
    V = _bf16_valued(rng, (B, NKV, S, HD))
    k_new = _bf16_valued(rng, (B, NKV, HD))
    v_new = _bf16_valued(rng, (B, NKV, HD))
    want = oatt.cpu_attention(q, K, V, positions, k_new, v_new)
    ctx = np.asarray(positions, np.int32) + 1
    mb = (S + 15) // 16
    tables = np.arange(B * mb, dtype=np.int32).reshape(B, mb)
    ck, cv = oatt.paged_from_dense(_bits(K), _bits(V), [S] * B, tables, B * mb)
    orc.cache_append(_bits(k_new), _bits(v_new), ck, cv, tables, ctx)
    got = orc.decode_attn(_bits(q), ck, cv, tables, ctx, 1 / math.sqrt(HD))
    np.testing.assert_allclose(got, want, rtol=1e-4, atol=1e-5)


def test_attention_special_cases():
    rng = np.random.default_rng(13)
    q, ck, cv, tables, _ = _attn_case(rng, 1, 4, 1, [32], 32)
    blk0 = tables[0, 0]
    # one key: the output is that key's value row exactly
    out = orc.decode_attn(q, ck, cv, tables, np.array([1], np.int32), 0.3)
    np.testing.assert_array_equal(out[0, 0], orc.bf16_widen(cv[blk0, 0, :, 0]))
    # identical keys: uniform weights -> the mean of the values
    rows = oatt.k_block_rows(ck)
    rows[tables[0, 0], 0] = rows[tables[0, 0], 0, 0]
    rows[tables[0, 1], 0] = rows[tables[0, 0], 0, 0]
    ck2 = oatt.k_block_tiled(rows)
    out = orc.decode_attn(q, ck2, cv, tables, np.array([32], np.int32), 0.3)
    vals = np.concatenate([orc.bf16_widen(cv[tables[0, j], 0]) for j in range(2)], axis=1)
    np.testing.assert_allclose(out[0, 0], vals.mean(axis=1), rtol=1e-6, atol=1e-6)


def test_cache_append_places_token():
    rng = np.random.default_rng(14)
    q, ck, cv, tables, ctx = _attn_case(rng, 2, 4, 2, [20, 33], 32)
    k_new = _bits(_bf16_valued(rng, (2, 2, 32)))
    v_new = _bits(_bf16_valued(rng, (2, 2, 32)))
    before = oatt.k_block_rows(ck)
    orc.cache_append(k_new, v_new, ck, cv, tables, ctx)
    rows = oatt.k_block_rows(ck)
    for b in range(2):
        t = ctx[b] - 1
        blk = tables[b, t // 16]
        np.testing.assert_array_equal(rows[blk, :, t % 16, :], k_new[b])
        before[blk, :, t % 16, :] = k_new[b]
        np.testing.assert_array_equal(cv[blk, :, :, t % 16], v_new[b])
    np.testing.assert_array_equal(rows, before)     # no other K element moved


def test_golden_attention():
    """Dense fixture (tests/golden/make_golden.py): the paged cache built from
    it and read by the C oracle reproduces cpu_layer's output."""
    z = np.load(os.path.join(GOLDEN, "attention_small.npz"))
    ck, cv = oatt.paged_from_dense(z["k_dense"], z["v_dense"], z["ctx"], z["tables"], 7)
    got = orc.decode_attn(z["q"], ck, cv, z["tables"], z["ctx"], float(z["scale"]))
    np.testing.assert_allclose(got, z["out"], rtol=1e-5, atol=1e-6)


# ------------------------------------------------------- K block layout ----
@pytest.mark.parametrize("D", [32, 64, 128, 256])
def test_k_block_layout_is_a_tiled_permutation(D):
    idx = oatt.k_block_index(D)
    assert sorted(idx.ravel().tolist()) == list(range(16 * D))           # a permutation
    assert (np.diff(idx, axis=1)[:, np.arange(D - 1) % 8 != 7] == 1).all()   # 8-dim runs
    # The QK tile reads: for tile t, dim group d0, its 8 tokens fill one 128-byte line.
    for t in (0, 1):
        toks = [s for s in range(16) if (s >> 2) & 1 == t]
        toks.sort(key=lambda s: (s >> 3) * 4 + (s & 3))
        for d0 in range(0, D, 8):
            starts = idx[toks, d0]
            assert starts[0] % 64 == 0 and (np.diff(starts) == 8).all()


def test_k_block_layout_matches_the_kernel_formula():
    """The formula the C oracle and the HIP kernels share, spelled out for a few
    (slot, d) against k_block_index."""
    D = 128
    idx = oatt.k_block_index(D)
    assert idx[0, 0] == 0 and idx[1, 0] == 8 and idx[3, 7] == 31
    assert idx[8, 0] == 32              # j8 = 4
    assert idx[4, 0] == 1024            # t = 1: after tile 0 (8 tokens x 128 dims)
    assert idx[0, 8] == 64              # g = 1
    assert idx[0, 32] == 256            # s = 1


# --------------------------------------------------------------- argmax ----
def test_argmax_matches_torch():
    rng = np.random.default_rng(15)
    x = _bits(_bf16_valued(rng, (6, 1000), scale=4))
    x[1, 10] = x[1, 900] = 0x4400                  # tie at 512.0: first index
    x[2, 333] = 0x7FC0                             # NaN ranks first
    want = torch.argmax(torch.from_numpy(x.view(np.int16)).view(torch.bfloat16), dim=1).numpy()
    np.testing.assert_array_equal(orc.greedy_argmax(x), want)
    assert orc.greedy_argmax(x)[1] == 10 and orc.greedy_argmax(x)[2] == 333
