"""ctypes binding of librngdpd.so, the HIP/gfx950 C ABI declared in include/rngdpd.h.

There is no fallback: if the library is missing or fails to load, every call
raises. Build it with ``python -c "import __graft_entry__ as g; g.build()"``
(or ``python -m rngd_pd_amd.build``).
"""
import ctypes
import os
import threading

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "librngdpd.so")

PDK_OK = 0
PDK_EHIP = -5
PDK_EAGAIN = -11
PDK_ENOMEM = -12
PDK_EINVAL = -22
PDK_ENOTSUP = -95
PDK_MAX_BATCH = 16
PDK_NOALLOC_SCRATCH_BYTES = 4 << 20
PDK_BLOCK_SIZE = 16
PDK_IPC_HANDLE_BYTES = 64
PDK_EVENT_TIMING = 0
PDK_EVENT_INTERPROCESS = 1
PDK_EVENT_SYNC = 2
PDK_COPY_D2H = 0
PDK_COPY_H2D = 1
PDK_COPY_D2D = 2
PDK_STREAM_READ = 0
PDK_STREAM_WRITE = 1
PDK_STREAM_COPY = 2
PDK_STREAM_NONTEMPORAL = 1


class PdkError(RuntimeError):
    """A librngdpd call failed; ``code`` is the negative status it returned."""

    def __init__(self, code, what, message):
        super().__init__(f"{what}: {message or 'error'} (status {code})")
        self.code = code


class PackReq(ctypes.Structure):
    _fields_ = [("src_k", ctypes.c_void_p), ("src_v", ctypes.c_void_p),
                ("frame", ctypes.c_void_p), ("layer_stride", ctypes.c_int64),
                ("tok_stride", ctypes.c_int64), ("P", ctypes.c_int32),
                ("flags", ctypes.c_int32)]


PDK_PACK_NARROW = 1
PDK_FRAME_K, PDK_FRAME_V, PDK_FRAME_KV = 1, 2, 3


class ScatterReq(ctypes.Structure):
    _fields_ = [("frame", ctypes.c_void_p), ("table", ctypes.c_void_p),
                ("P", ctypes.c_int32), ("n_table", ctypes.c_int32)]


_P = ctypes.c_void_p
_I = ctypes.c_int
_I64 = ctypes.c_int64
_U = ctypes.c_uintptr_t if hasattr(ctypes, "c_uintptr_t") else ctypes.c_size_t
_SZ = ctypes.c_size_t
_F = ctypes.c_float

# name -> (restype, argtypes); every declaration of include/rngdpd.h.
SIGNATURES = {
    "pdk_version": (_I, []),
    "pdk_last_error": (ctypes.c_char_p, []),
    "pdk_device_count": (_I, [ctypes.POINTER(_I)]),
    "pdk_set_device": (_I, [_I]),
    "pdk_pack_kv": (_I, [_P, _P, _I64, _I64, _I, _I, _I, _I, _I, _P, _U]),
    "pdk_pack_kv_batch": (_I, [ctypes.POINTER(PackReq), _I, _I, _I, _I, _I, _U]),
    "pdk_scatter_paged": (_I, [_P, _P, _I, _I, _I, _I, _I, _I, _P, _P, _I64, _I, _U]),
    "pdk_scatter_paged_batch": (_I, [ctypes.POINTER(ScatterReq), _I, _I, _I, _I, _I, _P, _P,
                                     _I64, _I, _U]),
    "pdk_scatter_paged_batch_counted": (_I, [ctypes.POINTER(ScatterReq), _I, _I, _I, _I, _I, _P,
                                             _P, _I64, _I, _P, _U]),
    "pdk_gather_paged": (_I, [_P, _P, _I64, _I, _P, _I, _I, _I, _I, _I, _I, _P, _U]),
    "pdk_decode_attn_workspace_bytes": (_SZ, [_I, _I, _I, _I]),
    "pdk_decode_attn": (_I, [_P, _P, _P, _I, _P, _I, _P, _I, _I, _I, _I, _I, ctypes.c_float,
                             _P, _SZ, _P, _U]),
    "pdk_decode_attn_noalloc": (_I, [_P, _P, _P, _I, _P, _I, _P, _I, _I, _I, _I, _I,
                                     ctypes.c_float, _P, _U]),
    "pdk_decode_attn_rope": (_I, [_P, _I, _P, _P, _P, _I, _P, _I, _P, _I, _I, _I, _I, _I,
                                  ctypes.c_float, _P, _SZ, _P, _I, _U]),
    "pdk_decode_attn_rope_rms": (_I, [_P, _I, _P, _I, ctypes.c_float, _P, _P, _P, _I, _P, _I,
                                      _P, _I, _I, _I, _I, _I, ctypes.c_float, _P, _SZ, _P, _I,
                                      _U]),
    "pdk_cache_append": (_I, [_P, _P, _P, _P, _I, _P, _I, _P, _I, _I, _I, _U]),
    "pdk_greedy_argmax": (_I, [_P, _I, _I, _I64, _P, _U]),
    "pdk_rmsnorm": (_I, [_P, _P, _P, _I, _I, ctypes.c_float, _P, _U]),
    "pdk_rope_cache_append": (_I, [_P, _I64, _P, _P, _P, _P, _I, _P, _P, _I, _I, _I, _I, _I,
                                   _U]),
    "pdk_rope_cache_append_partials": (_I, [_P, _I, _I, _P, _P, _P, _P, _I, _P, _P, _I, _I, _I,
                                            _I, _I, _U]),
    "pdk_rope_cache_append_partials_rms": (_I, [_P, _I, _I, _P, _I, ctypes.c_float, _P, _P, _P,
                                                _P, _I, _P, _P, _I, _I, _I, _I, _I, _U]),
    "pdk_swiglu": (_I, [_P, _I, _I, _P, _U]),
    "pdk_linear": (_I, [_P, _P, _I, _I, _I, _P, _P, _U]),
    "pdk_linear_swiglu": (_I, [_P, _P, _I, _I, _I, _P, _U]),
    "pdk_linear_splitk": (_I, [_P, _P, _I, _I, _I, _I, _P, _U]),
    "pdk_rmsnorm_partials": (_I, [_P, _P, _I, _P, _I, _I, ctypes.c_float, _P, _U]),
    "pdk_linear_argmax": (_I, [_P, _P, _I, _I, _I, _P, _P, _P, _U]),
    "pdk_weight_tiled_elems": (_I64, [_I, _I]),
    "pdk_weight_tile": (_I, [_P, _I, _I, _P, _U]),
    "pdk_linear_tiled": (_I, [_P, _P, _I, _I, _I, _P, _P, _U]),
    "pdk_linear_swiglu_tiled": (_I, [_P, _P, _I, _I, _I, _P, _U]),
    "pdk_linear_splitk_tiled": (_I, [_P, _P, _I, _I, _I, _I, _P, _U]),
    "pdk_linear_argmax_tiled": (_I, [_P, _P, _I, _I, _I, _P, _P, _P, _U]),
    "pdk_linear_ssq": (_I, [_P, _P, _I, _I, _I, _P, _P, _P, _U]),
    "pdk_linear_ssq_tiled": (_I, [_P, _P, _I, _I, _I, _P, _P, _P, _U]),
    "pdk_linear_swiglu_rms": (_I, [_P, _P, _I, _I, _I, _P, _I, _F, _P, _U]),
    "pdk_linear_swiglu_rms_tiled": (_I, [_P, _P, _I, _I, _I, _P, _I, _F, _P, _U]),
    "pdk_linear_splitk_rms": (_I, [_P, _P, _I, _I, _I, _I, _P, _I, _F, _P, _U]),
    "pdk_linear_splitk_rms_tiled": (_I, [_P, _P, _I, _I, _I, _I, _P, _I, _F, _P, _U]),
    "pdk_linear_splitk_final": (_I, [_P, _P, _I, _I, _I, _I, _P, _P, _P, _P, _U]),
    "pdk_linear_splitk_final_tiled": (_I, [_P, _P, _I, _I, _I, _I, _P, _P, _P, _P, _U]),
    "pdk_linear_argmax_rms": (_I, [_P, _P, _I, _I, _I, _P, _I, _F, _P, _P, _P, _U]),
    "pdk_linear_argmax_rms_tiled": (_I, [_P, _P, _I, _I, _I, _P, _I, _F, _P, _P, _P, _U]),
    "pdk_linear_ssq_xt": (_I, [_P, _P, _I, _I, _I, _P, _P, _P, _U]),
    "pdk_linear_swiglu_rms_xt": (_I, [_P, _P, _I, _I, _I, _P, _I, _F, _P, _U]),
    "pdk_linear_splitk_rms_xt": (_I, [_P, _P, _I, _I, _I, _I, _P, _I, _F, _P, _U]),
    "pdk_linear_splitk_final_xt": (_I, [_P, _P, _I, _I, _I, _I, _P, _P, _P, _P, _U]),
    "pdk_linear_argmax_rms_xt": (_I, [_P, _P, _I, _I, _I, _P, _I, _F, _P, _P, _P, _U]),
    "pdk_embed_ssq_xt": (_I, [_P, _I64, _P, _I, _I, _I, _P, _P, _U]),
    "pdk_decode_attn_rope_xt": (_I, [_P, _I, _P, _P, _P, _I, _P, _I, _P, _I, _I, _I, _I, _I,
                                     ctypes.c_float, _P, _SZ, _P, _I, _U]),
    "pdk_row_ssq": (_I, [_P, _I, _I, _P, _U]),
    "pdk_embed_ssq": (_I, [_P, _I64, _P, _I, _I, _I, _P, _P, _U]),
    "pdk_scatter_koni": (_I, [_P, _I64, _P, _I, _I, _P, _I, _P, _P, _I64, _I, _I, _I, _U]),
    "pdk_host_alloc": (_I, [_SZ, ctypes.POINTER(_P)]),
    "pdk_host_free": (_I, [_P]),
    "pdk_dev_alloc": (_I, [_SZ, ctypes.POINTER(_P)]),
    "pdk_dev_free": (_I, [_P]),
    "pdk_memcpy_d2h": (_I, [_P, _P, _SZ, _U]),
    "pdk_memcpy_h2d": (_I, [_P, _P, _SZ, _U]),
    "pdk_memcpy_d2d": (_I, [_P, _P, _SZ, _U]),
    "pdk_copy_kernel": (_I, [_P, _P, _SZ, _U]),
    "pdk_stream_probe": (_I, [_I, _P, _P, _SZ, _I, _I, ctypes.c_uint32, _P, _U]),
    "pdk_attn_read_probe": (_I, [_P, _P, _I, _P, _I, _P, _I, _I, _I, _I, _I, _P, _U]),
    "pdk_stream_create": (_I, [ctypes.POINTER(_U)]),
    "pdk_stream_destroy": (_I, [_U]),
    "pdk_stream_sync": (_I, [_U]),
    "pdk_event_create": (_I, [ctypes.POINTER(_U), _I]),
    "pdk_event_destroy": (_I, [_U]),
    "pdk_event_record": (_I, [_U, _U]),
    "pdk_event_query": (_I, [_U]),
    "pdk_event_sync": (_I, [_U]),
    "pdk_stream_wait_event": (_I, [_U, _U]),
    "pdk_event_elapsed_ms": (_I, [_U, _U, ctypes.POINTER(ctypes.c_float)]),
    "pdk_ipc_export_mem": (_I, [_P, _P]),
    "pdk_ipc_open_mem": (_I, [_P, ctypes.POINTER(_P)]),
    "pdk_ipc_close_mem": (_I, [_P]),
    "pdk_ipc_export_event": (_I, [_U, _P]),
    "pdk_ipc_open_event": (_I, [_P, ctypes.POINTER(_U)]),
    "pdk_pack_kv_layerwise": (_I, [ctypes.POINTER(PackReq), _I, _I, _I, _I, _I, _P, _U]),
    "pdk_copy_layers": (_I, [_P, _P, _SZ, _I, _I, _P, _P, _U]),
    "pdk_host_zero_frame_tail": (_I, [_P, _I, _I, _I, _I, _I, _I, _I]),
    "pdk_copy_frame_valid": (_I, [_P, _P, _I, _I, _I, _I, _I, _I, _I, _I, _U]),
    "pdk_scatter_paged_layerwise": (_I, [ctypes.POINTER(ScatterReq), _I, _I, _I, _I, _I, _P, _P,
                                         _I64, _I, _P, _U]),
}

_lib = None
_lock = threading.Lock()


def lib():
    """The loaded library with argtypes set; raises if it is not built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise RuntimeError(
                    f"librngdpd.so is not built ({LIB_PATH}); run __graft_entry__.build()")
            L = ctypes.CDLL(LIB_PATH)
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(L, name)
                fn.restype = res
                fn.argtypes = args
            _lib = L
    return _lib


def last_error():
    msg = lib().pdk_last_error()
    return msg.decode(errors="replace") if msg else ""


def check(rc, what):
    """Raise PdkError for a failing status; return PDK_OK / PDK_EAGAIN as is."""
    if rc == PDK_OK or rc == PDK_EAGAIN:
        return rc
    raise PdkError(rc, what, last_error())


def call(name, *args):
    return check(getattr(lib(), name)(*args), name)
