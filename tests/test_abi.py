"""librngdpd.so: it loads, exports every function include/rngdpd.h declares, and
rejects bad arguments with errno-style codes before touching a device."""
import ctypes
import os
import re

import pytest

from rngd_pd_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "rngdpd.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(pdk_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_api():
    names = declared_functions()
    for must in ("pdk_pack_kv", "pdk_scatter_paged", "pdk_decode_attn", "pdk_ipc_open_mem",
                 "pdk_last_error", "pdk_copy_layers"):
        assert must in names


def test_every_declared_symbol_is_exported_and_bound():
    lib = _lib.lib()
    for name in declared_functions():
        assert hasattr(lib, name), f"{name} is declared but not exported"
        assert name in _lib.SIGNATURES, f"{name} has no ctypes signature"
    assert set(_lib.SIGNATURES) <= set(declared_functions())


def test_version_and_constants():
    lib = _lib.lib()
    assert lib.pdk_version() == 100
    text = open(HEADER).read()
    for name in ("PDK_EINVAL", "PDK_ENOTSUP", "PDK_EHIP", "PDK_EAGAIN", "PDK_ENOMEM",
                 "PDK_MAX_BATCH", "PDK_BLOCK_SIZE", "PDK_PACK_NARROW", "PDK_COPY_H2D",
                 "PDK_FRAME_K", "PDK_FRAME_V", "PDK_FRAME_KV"):
        value = int(re.search(rf"#define {name}\s+\(?(-?\d+)", text).group(1))
        assert getattr(_lib, name) == value, name


def test_bad_arguments_return_einval_with_message():
    lib = _lib.lib()
    rc = lib.pdk_pack_kv(None, None, 0, 0, 1, 4, 16, 8, 128, None, 0)
    assert rc == _lib.PDK_EINVAL
    assert "frame" in _lib.last_error()
    buf = ctypes.create_string_buffer(64)
    ptr = (ctypes.addressof(buf) + 15) // 16 * 16
    rc = lib.pdk_pack_kv(ptr, ptr, 0, 1024, 1, 20, 16, 8, 128, ptr, 0)   # P > S
    assert rc == _lib.PDK_EINVAL and "P=20" in _lib.last_error()
    rc = lib.pdk_pack_kv(ptr, ptr, 0, 1024, 1, 4, 24, 8, 128, ptr, 0)    # S % 16
    assert rc == _lib.PDK_EINVAL
    rc = lib.pdk_pack_kv(ptr, ptr, 0, 1024, 1, 4, 16, 8, 96, ptr, 0)     # D % 64
    assert rc == _lib.PDK_ENOTSUP
    rc = lib.pdk_scatter_paged(ptr, ptr, 0, 1, 33, 64, 8, 128, ptr, ptr, 0, 10, 0)
    assert rc == _lib.PDK_EINVAL and "table" in _lib.last_error()


def test_decode_attn_argument_checks():
    lib = _lib.lib()
    buf = ctypes.create_string_buffer(64)
    p = (ctypes.addressof(buf) + 15) // 16 * 16
    call = lambda **kw: lib.pdk_decode_attn(  # noqa: E731
        p, p, p, kw.get("nb", 4), p, kw.get("mb", 4), p, kw.get("max_ctx", 64), kw.get("B", 2),
        kw.get("hq", 32), kw.get("hkv", 8), kw.get("d", 128), 1.0, None, 0, p, 0)
    assert call(d=64) == _lib.PDK_ENOTSUP
    assert call(hq=24) == _lib.PDK_ENOTSUP          # group 3
    assert call(hq=12) == _lib.PDK_EINVAL           # not a multiple of Hkv
    assert call(max_ctx=65) == _lib.PDK_EINVAL      # beyond max_blocks * 16
    assert call(B=0) == _lib.PDK_EINVAL
    # B*Hkv = 16 workgroups at 512 tokens: the launch splits and needs a workspace
    assert call(B=2, max_ctx=512, mb=32) == _lib.PDK_EINVAL and "workspace" in _lib.last_error()


@pytest.mark.parametrize("B,hq,ctx", [(16, 32, 512), (4, 32, 512), (1, 32, 2048), (3, 8, 1)])
def test_workspace_bound(B, hq, ctx):
    n = _lib.lib().pdk_decode_attn_workspace_bytes(B, hq, ctx, 128)
    splits = min(32, max(1, (ctx + 127) // 128))      # splits hold >= 128 tokens
    if splits == 1:
        assert n == 0
    else:
        assert n >= B * hq * splits * (128 + 2) * 4


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    monkeypatch.setattr(_lib, "_lib", None)
    monkeypatch.setattr(_lib, "LIB_PATH", str(tmp_path / "nope.so"))
    with pytest.raises(RuntimeError, match="not built"):
        _lib.lib()


NET_HEADER = os.path.join(ROOT, "include", "rngdpd_net.h")


def test_net_library_exports_its_header():
    """librngdpd_net.so (host-only tcp transport): every function of
    include/rngdpd_net.h is exported and bound; error codes agree."""
    from rngd_pd_amd.connector import tcp
    text = re.sub(r"/\*.*?\*/", "", open(NET_HEADER).read(), flags=re.S)
    names = sorted(set(re.findall(r"\b(pdk_[a-z0-9_]+)\s*\(", text)))
    assert "pdk_tcp_push" in names and "pdk_crc32" in names
    lib = tcp._net()
    for name in names:
        assert hasattr(lib, name), f"{name} is declared but not exported"
        assert getattr(lib, name).argtypes is not None, f"{name} has no ctypes signature"
    raw = open(NET_HEADER).read()
    for name, value in (("PDK_NET_ENOSPC", tcp.ENOSPC), ("PDK_NET_ETIMEDOUT", tcp.ETIMEDOUT),
                        ("PDK_NET_EIO", tcp.EIO)):
        assert int(re.search(rf"#define {name}\s+\((-?\d+)\)", raw).group(1)) == value
    assert lib.pdk_tcp_client_open(None, 1, 1.0, None) == -22


def test_host_zero_frame_tail_completes_a_narrow_frame():
    """The host's half of a frame the device filled narrow: what it leaves
    unwritten (K columns >= round16(P) or round64(P), V rows >= P) becomes zero,
    nothing else changes, and the frame equals the oracle's S-wide frame. Host
    memory only."""
    import ctypes
    import numpy as np
    from oracle import native as orc
    lib = _lib.lib()
    rng = np.random.default_rng(3)
    L, H, D, S = 3, 2, 64, 144
    for P in (0, 1, 7, 8, 9, 15, 16, 17, 63, 64, 65, 79, 129, 143, 144):
        k = rng.integers(0, 1 << 16, (L, S, H, D), dtype=np.uint16)
        v = rng.integers(0, 1 << 16, (L, S, H, D), dtype=np.uint16)
        want = orc.pack_kv(k, v, P, S)
        for k_round in (16, 64):
            frame = want.copy()
            kf = frame[:, 0].reshape(L, H * D, S)
            vf = frame[:, 1].reshape(L, H, S, D)
            k0 = min((P + k_round - 1) // k_round * k_round, S)
            kf[:, :, k0:] = 0xBEEF                    # what the device leaves unwritten
            vf[:, :, P:, :] = 0xBEEF
            for threads in (1, 4):
                f = frame.copy()
                rc = lib.pdk_host_zero_frame_tail(f.ctypes.data_as(ctypes.c_void_p), L, H, D, S,
                                                  P, k_round, threads)
                assert rc == 0, lib.pdk_last_error()
                np.testing.assert_array_equal(f, want,
                                              err_msg=f"P={P} k_round={k_round} threads={threads}")
    bad = np.zeros(16, np.uint16)
    assert lib.pdk_host_zero_frame_tail(bad.ctypes.data_as(ctypes.c_void_p), 1, 1, 8, 8, 9, 64,
                                        1) == _lib.PDK_EINVAL
    assert lib.pdk_host_zero_frame_tail(bad.ctypes.data_as(ctypes.c_void_p), 1, 1, 8, 8, 4, 32,
                                        1) == _lib.PDK_EINVAL


def test_decode_attn_refuses_contexts_past_its_limit():
    """max_ctx above 16384 (the header's limit) is refused before anything is
    launched; the pointers are never dereferenced, so placeholders do."""
    lib = _lib.lib()
    p = 1 << 20                                   # 16-byte aligned placeholder address
    rc = lib.pdk_decode_attn(p, p, p, 2048, p, 1100, p, 16400, 1, 32, 8, 128, 0.088, p, 1 << 30,
                             p, 0)
    assert rc == _lib.PDK_ENOTSUP
    assert "16384" in _lib.last_error()
