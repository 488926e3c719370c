"""Host logic of the same-GPU IPC transport (no GPU): selection by name and the
frame-slot life cycle driven by the consumer's ".done" files."""
import os
import threading
from collections import deque

import pytest

from rngd_pd_amd.connector import transport as T
from rngd_pd_amd.connector.ipc import IpcFramePool, IpcTransport, frame_nbytes


def test_selected_by_name(tmp_path, monkeypatch):
    monkeypatch.setenv("PD_SHM_ROOT", str(tmp_path))
    t = T.select_transport("ipc", root=str(tmp_path))
    assert isinstance(t, IpcTransport) and t.device_ipc and t.name == "ipc"
    assert isinstance(T.make_transport("ipc", root=str(tmp_path)), IpcTransport)
    # Byte blobs still use the shm file contract.
    t.push("r/layer.0/k", b"abc")
    assert t.pull("r/layer.0/k", timeout=1) == b"abc"
    assert os.path.exists(os.path.join(str(tmp_path), "r__layer.0__k"))


def _pool(tmp_path, n_slots):
    """An IpcFramePool without device memory: only its slot bookkeeping."""
    p = object.__new__(IpcFramePool)
    p.t = IpcTransport(str(tmp_path))
    p._free, p._out, p._lock = deque(range(n_slots)), {}, threading.Lock()
    return p


def test_slots_return_on_done_files(tmp_path):
    p = _pool(tmp_path, 2)
    a, b = p.acquire("a", timeout=0.01), p.acquire("b", timeout=0.01)
    assert {a, b} == {0, 1}
    with pytest.raises(TimeoutError, match="pool full"):
        p.acquire("c", timeout=0.02)
    p.t.push("a/ipc.done", b"1")                      # the consumer released a's slot
    assert p.acquire("c", timeout=0.5) == a
    assert not os.path.exists(p.t._path("a/ipc.done"))  # the producer deletes it
    assert set(p.outstanding()) == {"b", "c"}


def test_frame_size_and_ipc_limit():
    assert frame_nbytes(32, 8, 128, 512) == 64 << 20     # one Llama-3.1-8B request, S=512
    assert frame_nbytes(32, 8, 128, 2048) == 256 << 20
