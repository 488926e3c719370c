"""KONI token-block wire on the CPU: the header codec against the reference's
real-wire fixtures (tests/golden/koni, copied from tests/native_v4/fixtures),
the oracle receiver against the reference's transfer tests
(tests/native_v4/test_transfer.py, test_wire_boundary.py), and the product
receiver's validation against the oracle's."""
from pathlib import Path

import numpy as np
import pytest

from oracle import koni as ok
from rngd_pd_amd.connector import koni

GOLD = Path(__file__).parent / "golden" / "koni"


def test_fixtures_round_trip_byte_exact():
    for name, tag in (("ready.bin", 1), ("ack.bin", 3)):
        raw = (GOLD / name).read_bytes()
        m = koni.parse(raw)
        assert m["request_id"] == "native-probe-1"
        assert koni.control(tag, m["request_id"]) == raw
    raw = (GOLD / "handshake.bin").read_bytes()
    m = koni.parse(raw)
    assert m["layout"]["element_type"] == "Bfloat16" and m["aux"] is None
    assert koni.handshake(m["endpoint"], m["layout"]) == raw
    raw = (GOLD / "kv.bin").read_bytes()
    m = koni.parse(raw)
    assert [e["tensor"] for e in m["entries"]] == [0, 1, 2, 3]
    assert sum(e["bytes"] for e in m["entries"]) == 8192 and not m["is_final"]
    fast = koni.parse(raw, array_entries=True)
    np.testing.assert_array_equal(fast["entries"]["tensor"], [0, 1, 2, 3])
    assert koni.kv_message(m["request_id"], m["entries"], m["is_final"]) == raw
    assert koni.kv_message(m["request_id"], fast["entries"], False) == raw


def test_codec_round_trips():
    for rid in ["a", "abcdefg", "abcdefgh", "request-1234567890"]:
        assert koni.parse(koni.control(1, rid))["request_id"] == rid
        assert koni.parse(koni.pull(rid, [0, 1, 2]))["blocks"] == [0, 1, 2]
    assert koni.parse(koni.handshake("127.0.0.1:18422", koni.host_layout()))["layout"] == \
        koni.host_layout()
    m = koni.parse(koni.kv_message("r-long-request-id", [(0, 5, 3, 4096)], True))
    assert m["entries"] == [dict(tier=0, tensor=5, block=3, bytes=4096)] and m["is_final"]


def test_eight_byte_inline_string():
    for n in (1, 7, 8, 9, 16, 128):
        rid = "r" * n
        b = koni.control(3, rid)
        assert koni.parse(b)["request_id"] == rid
        if n <= 8:
            assert len(b) == 36 and b[8:8 + n] == rid.encode()
        assert koni.parse(koni.pull(rid, [0, 1]))["request_id"] == rid


def test_malformed_headers_and_cancel():
    assert koni.parse(koni.control(4, "cancel-request"))["kind"] == "cancel"
    for header in [b"", bytes(35), bytes(37), b"\xff" * 36]:
        with pytest.raises((koni.ProtocolError, UnicodeError)):
            koni.parse(header)
    with pytest.raises(koni.ProtocolError):
        koni.pull("x", [512])


def _msg(entries, final=False):
    return dict(kind="kv", request_id="test-long-request", entries=entries, is_final=final)


def _entry(t, b=0, n=1):
    return dict(tier=0, tensor=t, block=b, bytes=n * 2048)


def test_oracle_split_and_layout():
    r = ok.Receiver("test-long-request", 2)
    bits = np.arange(64 * 2 * 8 * 128, dtype=np.uint16).reshape(64, 2, 8, 128)
    raw = bits.astype("<u2").tobytes()
    entries = [_entry(t, n=2) for t in range(64)]
    assert r.accept(_msg(entries, True), [raw[:3], raw[3:2047], raw[2047:8193], raw[8193:]])
    expected = (bits.astype(np.uint32) << 16).view(np.float32)
    np.testing.assert_array_equal(r.keys.view(np.uint32),
                                  expected[::2].transpose(0, 2, 3, 1).view(np.uint32))
    np.testing.assert_array_equal(r.values.view(np.uint32),
                                  expected[1::2].transpose(0, 2, 1, 3).view(np.uint32))


class _View:
    """Enough of a PagedRequestView for the receiver's checks."""

    class cache:
        n_layers, n_kv_heads, head_dim = 32, 8, 128

    def __init__(self, n):
        self.num_tokens = n


def _both(n):
    return ok.Receiver("test-long-request", n), koni.KoniPagedReceiver("test-long-request", n, _View(n))


def _agree(recv_o, recv_p, message, frames):
    """Both receivers accept (the product only validates here) or both refuse."""
    try:
        recv_o.accept(message, frames)
        ok_o = True
    except ok.ProtocolError:
        ok_o = False
    try:
        rep_t, tok, _ = recv_p._validate(message, frames)
        recv_p.seen[rep_t, tok] = True
        recv_p.complete = bool(message["is_final"])
        ok_p = True
    except koni.ProtocolError:
        ok_p = False
    assert ok_o == ok_p, message["entries"]
    return ok_o


def test_reject_incomplete_duplicate_bounds_like_the_reference():
    o, p = _both(2)
    assert not _agree(o, p, _msg([_entry(0)], True), [bytes(2048)])      # incomplete final
    assert not o.seen.any() and not p.seen.any()
    assert _agree(o, p, _msg([_entry(0)]), [bytes(2048)])
    for entry in [_entry(0), _entry(64), _entry(1, b=2), _entry(1, n=3)]:
        assert not _agree(o, p, _msg([entry]), [bytes(entry["bytes"])])
    assert not _agree(o, p, _msg([_entry(1)]), [bytes(2047)])            # short payload
    assert not _agree(o, p, _msg([dict(tier=1, tensor=1, block=0, bytes=2048)]), [bytes(2048)])
    assert not _agree(o, p, dict(_msg([_entry(1)]), request_id="other"), [bytes(2048)])
    assert not _agree(o, p, _msg([_entry(1), _entry(1)]), [bytes(4096)])  # duplicate in batch
    rest = [_entry(t, b) for t in range(64) for b in range(2) if (t, b) != (0, 0)]
    assert _agree(o, p, _msg(rest, True), [bytes(2048 * len(rest))])
    assert not _agree(o, p, _msg([_entry(5)]), [bytes(2048)])            # already complete


def test_oracle_random_fragmentation_and_permuted_order():
    rng = np.random.default_rng(422)
    for n in (3, 1, 7):
        bits = rng.integers(0, 65536, size=(64, n, 8, 128), dtype=np.uint16)
        order = rng.permutation(64 * n)
        entries = [_entry(int(i // n), int(i % n)) for i in order]
        raw = b"".join(bits[i // n, i % n].astype("<u2").tobytes() for i in order)
        cuts = sorted(set([0, len(raw)] + rng.integers(0, len(raw), size=37).tolist()))
        frames = [raw[a:b] for a, b in zip(cuts, cuts[1:])]
        r = ok.Receiver("test-long-request", n)
        assert r.accept(_msg(entries, True), frames)
        expected = (bits.astype(np.uint32) << 16).view(np.float32)
        np.testing.assert_array_equal(r.keys.view(np.uint32),
                                      expected[::2].transpose(0, 2, 3, 1).view(np.uint32))
        np.testing.assert_array_equal(r.values.view(np.uint32),
                                      expected[1::2].transpose(0, 2, 1, 3).view(np.uint32))


def test_sender_payload_matches_entries():
    rng = np.random.default_rng(9)
    L, T = 2, 5
    k = rng.integers(0, 65536, (L, T, 8, 128), dtype=np.uint16)
    v = rng.integers(0, 65536, (L, T, 8, 128), dtype=np.uint16)
    entries = koni.koni_entries(L, 3, first_token=1)
    payload = koni.koni_payload(k, v, 1, 3)
    r = ok.Receiver("q", 4, n_layers=L)
    first = [_entry(t, 0) for t in range(2 * L)]
    head = b"".join((k if t % 2 == 0 else v)[t // 2, 0].astype("<u2").tobytes() for t in range(2 * L))
    r.accept(dict(kind="kv", request_id="q", entries=first, is_final=False), [head])
    assert r.accept(koni.parse(koni.kv_message("q", entries, True)), [payload])
    np.testing.assert_array_equal(r.keys.view(np.uint32),
                                  (k.astype(np.uint32) << 16)[:, :4].transpose(0, 2, 3, 1))
    np.testing.assert_array_equal(r.values.view(np.uint32),
                                  (v.astype(np.uint32) << 16)[:, :4].transpose(0, 2, 1, 3))
