"""Streams, events, pinned host buffers and same-GPU IPC handles over the C ABI.

Pinned memory is always allocated by the library (hipHostMalloc); existing
host memory is never registered. Objects free what they own on close() (and,
as a last resort, when collected).
"""
import ctypes

import numpy as np

from . import _lib
from ._lib import (PDK_EVENT_INTERPROCESS, PDK_EVENT_SYNC, PDK_EVENT_TIMING,
                   PDK_IPC_HANDLE_BYTES, PDK_OK, PDK_EAGAIN)

_U = _lib._U


class EventArray:
    """n HIP events as a ctypes uintptr array (pass ``.ptr`` to layer-wise calls)."""

    def __init__(self, n, flags=PDK_EVENT_SYNC):
        self.n = n
        self.arr = (_U * n)()
        for i in range(n):
            h = _U(0)
            _lib.call("pdk_event_create", ctypes.byref(h), flags)
            self.arr[i] = h.value

    @property
    def ptr(self):
        return ctypes.cast(self.arr, ctypes.c_void_p)

    def __getitem__(self, i):
        return self.arr[i]

    def sync(self, i=None):
        for j in (range(self.n) if i is None else [i]):
            _lib.call("pdk_event_sync", self.arr[j])

    def done(self, i):
        return _lib.call("pdk_event_query", self.arr[i]) == PDK_OK

    def close(self):
        if self.arr is not None:
            for i in range(self.n):
                if self.arr[i]:
                    _lib.lib().pdk_event_destroy(self.arr[i])
                    self.arr[i] = 0
            self.arr = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Event:
    """One HIP event (``timing=True`` for elapsed times)."""

    def __init__(self, flags=PDK_EVENT_TIMING, handle=None):
        self._owned = handle is None
        if handle is None:
            h = _U(0)
            _lib.call("pdk_event_create", ctypes.byref(h), flags)
            handle = h.value
        self.handle = handle

    def record(self, stream):
        _lib.call("pdk_event_record", self.handle, stream)

    def sync(self):
        _lib.call("pdk_event_sync", self.handle)

    def query(self):
        return _lib.call("pdk_event_query", self.handle) == PDK_OK

    def elapsed_ms(self, end):
        ms = ctypes.c_float(0)
        _lib.call("pdk_event_elapsed_ms", self.handle, end.handle, ctypes.byref(ms))
        return ms.value

    def ipc_handle(self):
        """64 opaque bytes another process opens with Event.from_ipc (interprocess events)."""
        buf = ctypes.create_string_buffer(PDK_IPC_HANDLE_BYTES)
        _lib.call("pdk_ipc_export_event", self.handle, buf)
        return buf.raw

    @classmethod
    def from_ipc(cls, handle_bytes):
        buf = ctypes.create_string_buffer(bytes(handle_bytes), PDK_IPC_HANDLE_BYTES)
        h = _U(0)
        _lib.call("pdk_ipc_open_event", buf, ctypes.byref(h))
        ev = cls(handle=h.value)
        ev._owned = True
        return ev

    def close(self):
        if self.handle and self._owned:
            _lib.lib().pdk_event_destroy(self.handle)
        self.handle = 0

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def stream_wait(stream, event_handle):
    _lib.call("pdk_stream_wait_event", stream, event_handle)


class PinnedBuffer:
    """Page-locked host memory from hipHostMalloc, viewable as numpy / memoryview."""

    def __init__(self, nbytes):
        self.nbytes = int(nbytes)
        p = ctypes.c_void_p(0)
        _lib.call("pdk_host_alloc", self.nbytes, ctypes.byref(p))
        self.ptr = p.value
        self._raw = (ctypes.c_uint8 * self.nbytes).from_address(self.ptr)

    def view(self, dtype=np.uint8, offset=0, count=None):
        arr = np.frombuffer(self._raw, dtype=np.uint8)[offset:]
        if count is not None:
            arr = arr[: count * np.dtype(dtype).itemsize]
        return arr.view(dtype)

    def memoryview(self, offset=0, nbytes=None):
        mv = memoryview(self._raw).cast("B")
        end = self.nbytes if nbytes is None else offset + nbytes
        return mv[offset:end]

    def close(self):
        if self.ptr:
            self._raw = None
            _lib.lib().pdk_host_free(ctypes.c_void_p(self.ptr))
            self.ptr = 0

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class DeviceBuffer:
    """A hipMalloc allocation of its own (exportable through IPC, < 2 GiB)."""

    def __init__(self, nbytes=None, ptr=None, owned=True, opened=False):
        if ptr is None:
            p = ctypes.c_void_p(0)
            _lib.call("pdk_dev_alloc", int(nbytes), ctypes.byref(p))
            ptr = p.value
        self.ptr = ptr
        self.nbytes = nbytes
        self._owned = owned
        self._opened = opened

    def ipc_handle(self):
        buf = ctypes.create_string_buffer(PDK_IPC_HANDLE_BYTES)
        _lib.call("pdk_ipc_export_mem", ctypes.c_void_p(self.ptr), buf)
        return buf.raw

    @classmethod
    def from_ipc(cls, handle_bytes, nbytes=None):
        buf = ctypes.create_string_buffer(bytes(handle_bytes), PDK_IPC_HANDLE_BYTES)
        p = ctypes.c_void_p(0)
        _lib.call("pdk_ipc_open_mem", buf, ctypes.byref(p))
        return cls(nbytes=nbytes, ptr=p.value, owned=False, opened=True)

    def close(self):
        if not self.ptr:
            return
        if self._opened:
            _lib.lib().pdk_ipc_close_mem(ctypes.c_void_p(self.ptr))
        elif self._owned:
            _lib.lib().pdk_dev_free(ctypes.c_void_p(self.ptr))
        self.ptr = 0

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def as_tensor(ptr, nbytes, device_index=0, dtype=None):
    """A torch tensor aliasing device memory at ``ptr`` (no copy, no ownership)."""
    import torch
    dtype = dtype or torch.bfloat16
    itemsize = torch.tensor([], dtype=dtype).element_size()
    n = nbytes // itemsize

    class _Holder:
        pass

    h = _Holder()
    h.__cuda_array_interface__ = {
        "shape": (n,), "typestr": "|u1" if dtype == torch.uint8 else "<i2",
        "data": (ptr, False), "version": 3, "strides": None,
    }
    t = torch.as_tensor(h, device=f"cuda:{device_index}")
    return t.view(dtype) if dtype != torch.uint8 else t
