"""torch-facing wrappers of the handoff kernels: pack, scatter, gather.

Shapes (bf16 CUDA tensors):
  prefill KV   k, v [L, T, Hkv, D] (or [T, Hkv, D] for one layer); any layer
               and token stride, [Hkv, D] contiguous. A stacked [L, 2, T, Hkv, D]
               tensor is passed as kv[:, 0], kv[:, 1].
  frame        [L, 2, Hkv*D*S]: per layer the K frame [Hkv, D, S] then the V
               frame [Hkv, S, D], columns >= P zero -- the bf16 payload the
               reference's ser() writes for that layer (connector/transport.py:29-37).
  paged cache  cache_k [L, nb, Hkv, 16, D], cache_v [L, nb, Hkv, D, 16]. A K block's
               16*D values are in the tiled token order of the C header (16-byte
               units of 8 dims of one token, ordered for the attention's QK reads);
               engines.paged_cache.k_block_rows converts a block to token rows.
"""
import ctypes

import torch

from .. import _lib
from .._lib import PackReq, ScatterReq, PDK_MAX_BATCH, PDK_BLOCK_SIZE

BF16 = torch.bfloat16


def stream_handle(stream=None):
    """hipStream_t of a torch stream (default: the current stream) as an int."""
    if stream is None:
        return torch.cuda.current_stream().cuda_stream
    if isinstance(stream, int):
        return stream
    return stream.cuda_stream


def _need(t, name, dtype=BF16):
    if not isinstance(t, torch.Tensor) or not t.is_cuda:
        raise TypeError(f"{name} must be a CUDA tensor")
    if t.dtype != dtype:
        raise TypeError(f"{name} must be {dtype}, got {t.dtype}")


def frame_shape(n_layers, n_kv_heads, head_dim, S):
    return (n_layers, 2, n_kv_heads * head_dim * S)


def frame_views(frame, layer, n_kv_heads, head_dim, S):
    """(k [Hkv, D, S], v [Hkv, S, D]) views of one layer of a frame tensor."""
    return (frame[layer, 0].view(n_kv_heads, head_dim, S),
            frame[layer, 1].view(n_kv_heads, S, head_dim))


def _as_layers(k, v):
    if k.dim() == 3:
        k, v = k.unsqueeze(0), v.unsqueeze(0)
    if k.dim() != 4 or k.shape != v.shape:
        raise ValueError(f"k/v must be [L, T, Hkv, D] of equal shape, got {tuple(k.shape)} "
                         f"and {tuple(v.shape)}")
    L, T, H, D = k.shape
    for name, t in (("k", k), ("v", v)):
        if t.stride(3) != 1 or t.stride(2) != D:
            raise ValueError(f"{name}: [Hkv, D] must be contiguous per token")
    if k.stride(0) != v.stride(0) or k.stride(1) != v.stride(1):
        raise ValueError("k and v must share layer and token strides")
    return k, v


def pack_kv(k, v, num_tokens, S, frame=None, stream=None, frame_ptr=None, narrow=False):
    """Pack the first ``num_tokens`` tokens of every layer into an S-wide frame.

    Replaces engines/prefill_full.py:378-382 (zero-pad to S, download) and the
    bf16 encode of connector/transport.py:33-35. ``frame_ptr`` (instead of
    ``frame``) packs into any device-visible memory of the frame's size, such
    as a pinned host buffer: the kernel's own stores then carry the download,
    with no staging copy. ``narrow`` leaves the columns >= num_tokens unwritten,
    for a consumer that reads only the valid columns (the same-GPU scatter).
    Returns the frame tensor, or None with frame_ptr."""
    _need(k, "k")
    _need(v, "v")
    k, v = _as_layers(k, v)
    L, T, H, D = k.shape
    if not 0 <= num_tokens <= min(T, S):
        raise ValueError(f"num_tokens={num_tokens} outside [0, min(T={T}, S={S})]")
    if frame_ptr is not None:
        if frame is not None:
            raise ValueError("pass frame or frame_ptr, not both")
        ptr = int(frame_ptr)
    else:
        if frame is None:
            frame = torch.empty(frame_shape(L, H, D, S), dtype=BF16, device=k.device)
        elif tuple(frame.shape) != frame_shape(L, H, D, S) or not frame.is_contiguous():
            raise ValueError(f"frame must be contiguous {frame_shape(L, H, D, S)}")
        ptr = frame.data_ptr()
    req = PackReq(k.data_ptr(), v.data_ptr(), ptr, k.stride(0), k.stride(1), int(num_tokens),
                  _lib.PDK_PACK_NARROW if narrow else 0)
    _lib.call("pdk_pack_kv_batch", ctypes.byref(req), 1, L, S, H, D, stream_handle(stream))
    return frame


def pack_kv_batch(reqs, S, narrow=False, stream=None):
    """reqs: list of (k, v, num_tokens, frame) with equal (L, Hkv, D); frames
    preallocated [L, 2, Hkv*D*S]. Launches ceil(n/16) kernels. ``narrow``
    leaves columns >= num_tokens unwritten (device-only consumers)."""
    if not reqs:
        return
    L = H = D = None
    arr = []
    for k, v, P, frame in reqs:
        _need(k, "k")
        _need(v, "v")
        k, v = _as_layers(k, v)
        if L is None:
            L, _, H, D = k.shape
        if (k.shape[0], k.shape[2], k.shape[3]) != (L, H, D):
            raise ValueError("all requests of a batch must share (L, Hkv, D)")
        if not 0 <= P <= min(k.shape[1], S):
            raise ValueError(f"num_tokens={P} outside [0, min(T, S)]")
        if tuple(frame.shape) != frame_shape(L, H, D, S) or not frame.is_contiguous():
            raise ValueError(f"frame must be contiguous {frame_shape(L, H, D, S)}")
        arr.append(PackReq(k.data_ptr(), v.data_ptr(), frame.data_ptr(), k.stride(0),
                           k.stride(1), int(P), _lib.PDK_PACK_NARROW if narrow else 0))
    st = stream_handle(stream)
    for i in range(0, len(arr), PDK_MAX_BATCH):
        chunk = arr[i:i + PDK_MAX_BATCH]
        c_arr = (PackReq * len(chunk))(*chunk)
        _lib.call("pdk_pack_kv_batch", c_arr, len(chunk), L, S, H, D, st)


def _check_cache(cache_k, cache_v):
    _need(cache_k, "cache_k")
    _need(cache_v, "cache_v")
    if cache_k.dim() == 4:
        cache_k, cache_v = cache_k.unsqueeze(0), cache_v.unsqueeze(0)
    L, nb, H, bs, D = cache_k.shape
    if bs != PDK_BLOCK_SIZE or tuple(cache_v.shape) != (L, nb, H, D, bs):
        raise ValueError(f"cache_k must be [L, nb, Hkv, 16, D] and cache_v [L, nb, Hkv, D, 16]; "
                         f"got {tuple(cache_k.shape)}, {tuple(cache_v.shape)}")
    if not (cache_k.is_contiguous() and cache_v.is_contiguous()):
        raise ValueError("paged caches must be contiguous")
    return cache_k, cache_v


def _table_tensor(table, device):
    """A validated device int32 block table; host inputs are checked first."""
    if isinstance(table, torch.Tensor) and table.is_cuda:
        if table.dtype != torch.int32 or not table.is_contiguous():
            raise TypeError("device block table must be contiguous int32")
        return table
    t = torch.as_tensor(table, dtype=torch.int32).contiguous()
    return t.to(device, non_blocking=False)


def validate_table(table, P, num_blocks):
    """Host check of a block table before it reaches the kernel."""
    t = torch.as_tensor(table).to("cpu", torch.int64)
    need = (P + PDK_BLOCK_SIZE - 1) // PDK_BLOCK_SIZE
    if t.numel() < need:
        raise ValueError(f"block table has {t.numel()} entries, {P} tokens need {need}")
    head = t[:need]
    if need and (int(head.min()) < 0 or int(head.max()) >= num_blocks):
        raise ValueError(f"block ids must lie in [0, {num_blocks})")


def scatter_paged(frame, block_table, num_tokens, S, cache_k, cache_v, n_kv_heads=None,
                  head_dim=None, stream=None):
    """Place tokens 0..num_tokens-1 of every layer of ``frame`` into the paged cache.

    Replaces connector/rngd_kv.py:160-165 and engines/decode_batch.py:305-377."""
    cache_k, cache_v = _check_cache(cache_k, cache_v)
    L, nb, H, _, D = cache_k.shape
    _need(frame, "frame")
    if tuple(frame.shape) != frame_shape(L, H, D, S) or not frame.is_contiguous():
        raise ValueError(f"frame must be contiguous {frame_shape(L, H, D, S)}")
    if not (isinstance(block_table, torch.Tensor) and block_table.is_cuda):
        validate_table(block_table, num_tokens, nb)
    table = _table_tensor(block_table, frame.device)
    _lib.call("pdk_scatter_paged", frame.data_ptr(), table.data_ptr(), table.numel(), L,
              int(num_tokens), S, H, D, cache_k.data_ptr(), cache_v.data_ptr(),
              cache_k.stride(0), nb, stream_handle(stream))


def scatter_paged_batch(reqs, S, cache_k, cache_v, stream=None, skipped=None):
    """reqs: list of (frame, device int32 table, num_tokens).

    Block ids outside [0, num_blocks) are skipped by the kernel. ``skipped``
    (a device int32 tensor of one element): the calls add the number of
    skipped ids to it, with no host synchronisation; read it once the stream
    has passed them (nonzero: some KV was not placed). check_skipped() does
    that read and raises."""
    cache_k, cache_v = _check_cache(cache_k, cache_v)
    L, nb, H, _, D = cache_k.shape
    arr = []
    for frame, table, P in reqs:
        _need(frame, "frame")
        if tuple(frame.shape) != frame_shape(L, H, D, S) or not frame.is_contiguous():
            raise ValueError(f"frame must be contiguous {frame_shape(L, H, D, S)}")
        _need(table, "table", torch.int32)
        arr.append(ScatterReq(frame.data_ptr(), table.data_ptr(), int(P), table.numel()))
    if skipped is not None:
        _need(skipped, "skipped", torch.int32)
    st = stream_handle(stream)
    for i in range(0, len(arr), PDK_MAX_BATCH):
        chunk = arr[i:i + PDK_MAX_BATCH]
        c_arr = (ScatterReq * len(chunk))(*chunk)
        if skipped is None:
            _lib.call("pdk_scatter_paged_batch", c_arr, len(chunk), L, S, H, D,
                      cache_k.data_ptr(), cache_v.data_ptr(), cache_k.stride(0), nb, st)
        else:
            _lib.call("pdk_scatter_paged_batch_counted", c_arr, len(chunk), L, S, H, D,
                      cache_k.data_ptr(), cache_v.data_ptr(), cache_k.stride(0), nb,
                      skipped.data_ptr(), st)


def check_skipped(skipped, stream=None):
    """Wait for ``stream`` (default: the current one) and raise ValueError if
    the counted scatters before it skipped any block id."""
    (stream or torch.cuda.current_stream(skipped.device)).synchronize()
    n = int(skipped.item())
    if n:
        raise ValueError(f"{n} block ids outside [0, num_blocks): their tokens were not placed")


def gather_paged(cache_k, cache_v, block_table, num_tokens, S, frame=None, stream=None):
    """Inverse of scatter_paged: an S-wide frame of the request (zero for t >= P)."""
    cache_k, cache_v = _check_cache(cache_k, cache_v)
    L, nb, H, _, D = cache_k.shape
    if not (isinstance(block_table, torch.Tensor) and block_table.is_cuda):
        validate_table(block_table, num_tokens, nb)
    table = _table_tensor(block_table, cache_k.device)
    if frame is None:
        frame = torch.empty(frame_shape(L, H, D, S), dtype=BF16, device=cache_k.device)
    _lib.call("pdk_gather_paged", cache_k.data_ptr(), cache_v.data_ptr(), cache_k.stride(0), nb,
              table.data_ptr(), table.numel(), L, int(num_tokens), S, H, D, frame.data_ptr(),
              stream_handle(stream))
    return frame


def copy_kernel(dst, src, stream=None):
    """Plain 16-byte-vector device copy (traffic-counter calibration)."""
    n = src.numel() * src.element_size()
    _lib.call("pdk_copy_kernel", dst.data_ptr(), src.data_ptr(), n, stream_handle(stream))



_SINKS = {}


def stream_probe(kind, dst=None, src=None, nbytes=None, nontemporal=False, blocks=0,
                 key=0x9E3779B9, stream=None):
    """One streaming-probe launch: kind "read" (src), "write" (dst) or "copy".
    blocks=0 is one-shot (one 16-byte vector per lane, a workgroup per 4 KiB);
    blocks>0 a grid-stride loop over that many workgroups. A read stores
    nothing in practice (a word lands in a 1 KiB per-device sink only where its
    fold equals ``key``)."""
    kinds = {"read": _lib.PDK_STREAM_READ, "write": _lib.PDK_STREAM_WRITE,
             "copy": _lib.PDK_STREAM_COPY}
    t = src if src is not None else dst
    dev = t.device
    sink = _SINKS.get(dev)
    if sink is None:
        sink = _SINKS[dev] = torch.zeros(256, dtype=torch.int32, device=dev)
    if nbytes is None:
        nbytes = t.numel() * t.element_size()
    _lib.call("pdk_stream_probe", kinds[kind], dst.data_ptr() if dst is not None else None,
              src.data_ptr() if src is not None else None, int(nbytes),
              _lib.PDK_STREAM_NONTEMPORAL if nontemporal else 0, int(blocks), key & 0xFFFFFFFF,
              sink.data_ptr(), stream_handle(stream))
