"""The bf16 wire of the /dev/shm handoff.

ser/deser keep the reference's format (connector/transport.py:25-43): a bf16
blob is ``pickle.dumps({"bf16": u16, "shape": shape}, protocol=4)`` where u16 is
the high half of each float32 (truncation), and deser widens it back. deser
reads blobs with a restricted unpickler that can only rebuild numpy arrays,
so a file dropped into the shared directory cannot execute code.

The frame codec writes and reads the same bytes without building the blob:
the pickle envelope of a bf16 frame depends only on the frame's shape (and the
numpy version doing the pickling), so it is captured once per shape by
pickling a marker array and splitting around its payload. A sender writes
header + payload + trailer straight from a pinned staging buffer (os.writev);
a receiver checks header and trailer against the envelope it expects and DMAs
the payload in place. Anything else falls back to the restricted unpickler.
"""
import io
import math
import pickle
import threading

import numpy as np

WIRE = "fp16"        # module default, as in the reference; serving sets "bf16"


class _NumpyOnlyUnpickler(pickle.Unpickler):
    """Unpickler that resolves only the globals a numpy array pickle names."""

    ALLOWED = {
        ("numpy._core.multiarray", "_reconstruct"),
        ("numpy.core.multiarray", "_reconstruct"),
        ("numpy", "ndarray"),
        ("numpy", "dtype"),
    }

    def find_class(self, module, name):
        if (module, name) in self.ALLOWED:
            return super().find_class(module, name)
        raise pickle.UnpicklingError(f"blob names {module}.{name}; only numpy arrays are accepted")


def safe_loads(buf):
    return _NumpyOnlyUnpickler(io.BytesIO(buf)).load()


def ser(arr, wire=None):
    """float array -> wire blob (connector/transport.py:29-37)."""
    a = np.ascontiguousarray(arr)
    if (wire or WIRE) == "bf16":
        f = a if a.dtype == np.float32 else a.astype(np.float32)
        u = (f.view(np.uint32) >> 16).astype(np.uint16)
        return pickle.dumps({"bf16": u, "shape": a.shape}, protocol=4)
    return pickle.dumps(a.astype(np.float16), protocol=4)


def deser(buf):
    """wire blob -> float32 array (connector/transport.py:39-43)."""
    o = safe_loads(buf)
    if isinstance(o, dict) and "bf16" in o:
        u = np.asarray(o["bf16"])
        if u.dtype != np.uint16:
            raise ValueError(f"bf16 payload has dtype {u.dtype}")
        return (u.astype(np.uint32) << 16).view(np.float32).reshape(o["shape"])
    if not isinstance(o, np.ndarray):
        raise ValueError(f"blob holds {type(o).__name__}, not an array")
    return o.astype(np.float32)


_ENV_LOCK = threading.Lock()
_ENVELOPES = {}
MIN_SPLIT_BYTES = 256     # smaller payloads are simply pickled whole


def envelope(shape):
    """(header, trailer) bytes around the payload of a bf16 blob of ``shape``."""
    shape = tuple(int(x) for x in shape)
    env = _ENVELOPES.get(shape)
    if env is not None:
        return env
    n = math.prod(shape)
    if n * 2 < MIN_SPLIT_BYTES:
        raise ValueError(f"payload of {n * 2} bytes is below the split threshold")
    for salt in range(1, 64):
        marker = ((np.arange(n, dtype=np.uint64) * (2654435761 + salt) + salt) >> 7).astype(np.uint16)
        payload = marker.tobytes()
        blob = pickle.dumps({"bf16": marker.reshape(shape), "shape": tuple(shape)}, protocol=4)
        off = blob.find(payload)
        if off >= 0 and blob.find(payload, off + 1) < 0:
            env = (blob[:off], blob[off + len(payload):])
            with _ENV_LOCK:
                _ENVELOPES[shape] = env
            return env
    raise RuntimeError(f"could not isolate the pickle envelope of shape {shape}")


def encode_parts(payload, shape):
    """[header, payload, trailer]: the bytes of ser(x, "bf16") for the bf16 bits
    ``payload`` (a bytes-like object of prod(shape)*2 bytes) without copying it."""
    shape = tuple(int(x) for x in shape)
    nbytes = math.prod(shape) * 2
    mv = memoryview(payload).cast("B")
    if len(mv) != nbytes:
        raise ValueError(f"payload has {len(mv)} bytes, shape {shape} needs {nbytes}")
    if nbytes < MIN_SPLIT_BYTES:
        u = np.frombuffer(mv, dtype=np.uint16).reshape(shape)
        return [pickle.dumps({"bf16": u.copy(), "shape": shape}, protocol=4)]
    header, trailer = envelope(shape)
    return [header, mv, trailer]


def payload_range(buf, shape):
    """(offset, nbytes) of the payload if ``buf`` is exactly the envelope this
    process writes for ``shape``; None otherwise (use decode_payload)."""
    shape = tuple(int(x) for x in shape)
    nbytes = math.prod(shape) * 2
    if nbytes < MIN_SPLIT_BYTES:
        return None
    header, trailer = envelope(shape)
    mv = memoryview(buf).cast("B")
    if len(mv) != len(header) + nbytes + len(trailer):
        return None
    if mv[:len(header)] != header or mv[len(mv) - len(trailer):] != trailer:
        return None
    return len(header), nbytes


def decode_payload(buf, shape=None):
    """uint16 bf16 bits of a bf16 blob (via the restricted unpickler)."""
    o = safe_loads(buf)
    if not (isinstance(o, dict) and "bf16" in o):
        raise ValueError("not a bf16 wire blob")
    u = np.asarray(o["bf16"])
    if u.dtype != np.uint16:
        raise ValueError(f"bf16 payload has dtype {u.dtype}")
    if shape is not None and tuple(o["shape"]) != tuple(shape):
        raise ValueError(f"blob shape {tuple(o['shape'])} differs from the expected {tuple(shape)}")
    return np.ascontiguousarray(u).reshape(o["shape"])
