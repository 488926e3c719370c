"""ctypes wrapper over liboracle.so -- TEST INFRASTRUCTURE (see oracle/__init__.py).

Arrays are numpy; bf16 tensors are numpy uint16 bit patterns.
"""
import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib = None

_P = ctypes.c_void_p
_I = ctypes.c_int
_I64 = ctypes.c_int64


def build():
    """Compile pdk_oracle.c with the committed Makefile."""
    subprocess.run(["make", "-C", _HERE, "-B", "liboracle.so"], check=True,
                   stdout=subprocess.PIPE, stderr=subprocess.STDOUT)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = ctypes.CDLL(LIB_PATH)
        sigs = {
            "orc_bf16_truncate": [_P, _I64, _P],
            "orc_bf16_widen": [_P, _I64, _P],
            "orc_pack_kv": [_P, _P, _I64, _I64, _I, _I, _I, _I, _I, _P],
            "orc_scatter_paged": [_P, _P, _I, _I, _I, _I, _I, _I, _P, _P, _I64, _I],
            "orc_gather_paged": [_P, _P, _I64, _I, _P, _I, _I, _I, _I, _I, _I, _P],
            "orc_cache_append": [_P, _P, _P, _P, _I, _P, _I, _P, _I, _I, _I],
            "orc_decode_attn": [_P, _P, _P, _I, _P, _I, _P, _I, _I, _I, _I, ctypes.c_float, _P],
            "orc_greedy_argmax": [_P, _I, _I, _I64, _P],
        }
        for name, args in sigs.items():
            fn = getattr(L, name)
            fn.argtypes = args
            fn.restype = None if name.startswith("orc_bf16") else _I
        _lib = L
    return _lib


def _ptr(a):
    return a.ctypes.data_as(ctypes.c_void_p)


def _check(rc, what):
    if rc != 0:
        raise ValueError(f"{what} failed with {rc}")


def bf16_truncate(x):
    x = np.ascontiguousarray(x, np.float32)
    out = np.empty(x.shape, np.uint16)
    lib().orc_bf16_truncate(_ptr(x), x.size, _ptr(out))
    return out


def bf16_widen(u):
    u = np.ascontiguousarray(u, np.uint16)
    out = np.empty(u.shape, np.float32)
    lib().orc_bf16_widen(_ptr(u), u.size, _ptr(out))
    return out


def pack_kv(src_k, src_v, P, S):
    """src_k/src_v: uint16 [L, T, Hkv, D] (contiguous). Returns frame [L, 2, Hkv*D*S]."""
    src_k = np.ascontiguousarray(src_k, np.uint16)
    src_v = np.ascontiguousarray(src_v, np.uint16)
    L, T, H, D = src_k.shape
    frame = np.empty((L, 2, H * D * S), np.uint16)
    _check(lib().orc_pack_kv(_ptr(src_k), _ptr(src_v), T * H * D, H * D, L, P, S, H, D,
                             _ptr(frame)), "orc_pack_kv")
    return frame


def scatter_paged(frame, table, P, S, H, D, cache_k, cache_v):
    """In place into cache_k [L, nb, H, 16, D] / cache_v [L, nb, H, D, 16]."""
    frame = np.ascontiguousarray(frame, np.uint16)
    table = np.ascontiguousarray(table, np.int32)
    L, nb = cache_k.shape[0], cache_k.shape[1]
    assert cache_k.flags.c_contiguous and cache_v.flags.c_contiguous
    _check(lib().orc_scatter_paged(_ptr(frame), _ptr(table), len(table), L, P, S, H, D,
                                   _ptr(cache_k), _ptr(cache_v), nb * H * 16 * D, nb),
           "orc_scatter_paged")


def gather_paged(cache_k, cache_v, table, P, S):
    L, nb, H, _, D = cache_k.shape
    table = np.ascontiguousarray(table, np.int32)
    frame = np.empty((L, 2, H * D * S), np.uint16)
    _check(lib().orc_gather_paged(_ptr(np.ascontiguousarray(cache_k)), _ptr(np.ascontiguousarray(cache_v)),
                                  nb * H * 16 * D, nb, _ptr(table), len(table), L, P, S, H, D,
                                  _ptr(frame)), "orc_gather_paged")
    return frame


def cache_append(k_new, v_new, cache_k, cache_v, tables, ctx):
    """cache_k [nb, H, 16, D], cache_v [nb, H, D, 16] (one layer), in place."""
    k_new = np.ascontiguousarray(k_new, np.uint16)
    v_new = np.ascontiguousarray(v_new, np.uint16)
    tables = np.ascontiguousarray(tables, np.int32)
    ctx = np.ascontiguousarray(ctx, np.int32)
    nb, H, _, D = cache_k.shape
    B = k_new.shape[0]
    _check(lib().orc_cache_append(_ptr(k_new), _ptr(v_new), _ptr(cache_k), _ptr(cache_v), nb,
                                  _ptr(tables), tables.shape[1], _ptr(ctx), B, H, D),
           "orc_cache_append")


def decode_attn(q, cache_k, cache_v, tables, ctx, scale):
    """q uint16 [B, Hq, D]; one layer's paged cache. Returns float32 [B, Hq, D]."""
    q = np.ascontiguousarray(q, np.uint16)
    tables = np.ascontiguousarray(tables, np.int32)
    ctx = np.ascontiguousarray(ctx, np.int32)
    B, Hq, D = q.shape
    nb, H = cache_k.shape[0], cache_k.shape[1]
    out = np.empty((B, Hq, D), np.float32)
    _check(lib().orc_decode_attn(_ptr(q), _ptr(np.ascontiguousarray(cache_k)),
                                 _ptr(np.ascontiguousarray(cache_v)), nb, _ptr(tables),
                                 tables.shape[1], _ptr(ctx), B, Hq, H, D, float(scale), _ptr(out)),
           "orc_decode_attn")
    return out


def greedy_argmax(logits_u16):
    x = np.ascontiguousarray(logits_u16, np.uint16)
    B, V = x.shape
    out = np.empty(B, np.int32)
    _check(lib().orc_greedy_argmax(_ptr(x), B, V, V, _ptr(out)), "orc_greedy_argmax")
    return out
