"""The product's wire codec against the oracle's restatement of ser/deser."""
import os
import pickle

import numpy as np
import pytest

from oracle import wire as owire
from rngd_pd_amd.connector import transport as kv
from rngd_pd_amd.connector import wire


def _bf16_valued(seed, shape):
    x = np.random.default_rng(seed).standard_normal(shape).astype(np.float32)
    return (x.view(np.uint32) >> 16 << 16).view(np.float32)


@pytest.mark.parametrize("shape", [(8, 128, 512), (8, 512, 128), (8, 16, 128), (2, 2, 4, 2, 8),
                                   (3,), (1, 2, 3)])
def test_ser_identical_to_reference(shape):
    x = np.random.default_rng(sum(shape)).standard_normal(shape).astype(np.float32)
    assert wire.ser(x, "bf16") == owire.ser(x, "bf16")
    assert wire.ser(x, "fp16") == owire.ser(x, "fp16")


@pytest.mark.parametrize("shape", [(8, 128, 512), (8, 512, 128), (2, 64, 16), (8, 16, 128)])
def test_encode_parts_byte_exact(shape):
    x = _bf16_valued(len(shape), shape)
    u = (x.view(np.uint32) >> 16).astype(np.uint16)
    parts = wire.encode_parts(u.tobytes(), shape)
    assert b"".join(bytes(p) for p in parts) == owire.ser(x, "bf16")


def test_small_payload_is_pickled_whole():
    x = _bf16_valued(1, (2, 3))
    u = (x.view(np.uint32) >> 16).astype(np.uint16)
    parts = wire.encode_parts(u.tobytes(), (2, 3))
    assert len(parts) == 1 and parts[0] == owire.ser(x, "bf16")


def test_payload_range_and_decode():
    shape = (8, 16, 128)
    x = _bf16_valued(2, shape)
    blob = owire.ser(x, "bf16")
    off, n = wire.payload_range(blob, shape)
    u = (x.view(np.uint32) >> 16).astype(np.uint16)
    assert blob[off:off + n] == u.tobytes()
    assert wire.payload_range(blob, (8, 128, 16)) is None          # another shape
    assert wire.payload_range(blob[:-1], shape) is None            # short file
    np.testing.assert_array_equal(wire.decode_payload(blob, shape), u)
    with pytest.raises(ValueError):
        wire.decode_payload(blob, (16, 8, 128))


def test_deser_matches_reference_and_numpy1_envelope():
    x = np.random.default_rng(3).standard_normal((4, 5, 6)).astype(np.float32)
    blob = owire.ser(x, "bf16")
    np.testing.assert_array_equal(wire.deser(blob), owire.deser(blob))
    # A writer on numpy 1.x names numpy.core.multiarray; it is still accepted.
    # Rewrite the SHORT_BINUNICODE (length byte) and the first FRAME length.
    new_name, old_name = b"\x8c\x16numpy._core.multiarray", b"\x8c\x15numpy.core.multiarray"
    if new_name in blob and blob[2:3] == b"\x95":
        old = blob.replace(new_name, old_name, 1)
        frame_len = int.from_bytes(old[3:11], "little") - 1
        old = old[:3] + frame_len.to_bytes(8, "little") + old[11:]
        np.testing.assert_array_equal(wire.deser(old), owire.deser(blob))


def test_deser_refuses_code():
    class Evil:
        def __reduce__(self):
            return (os.system, ("echo pwned",))
    with pytest.raises(pickle.UnpicklingError):
        wire.deser(pickle.dumps(Evil(), protocol=4))
    with pytest.raises(pickle.UnpicklingError):
        wire.deser(pickle.dumps({"bf16": Evil(), "shape": (1,)}, protocol=4))


def test_transport_module_wire_default():
    """kv.WIRE defaults to fp16 and ser() follows it, as the reference's module does."""
    x = np.random.default_rng(0).standard_normal((8, 16, 128)).astype(np.float32)
    old = kv.WIRE
    try:
        assert kv.WIRE == "fp16"
        assert kv.ser(x) == owire.ser(x, "fp16")
        kv.WIRE = "bf16"
        assert kv.ser(x) == owire.ser(x, "bf16")
        assert kv.ser(x, wire="fp16") == owire.ser(x, "fp16")
    finally:
        kv.WIRE = old
