"""RngdKVConnector: the vLLM KVConnector v1 surface of the prefill->decode handoff.

Same surface and key scheme as the reference (connector/rngd_kv.py:27-169):
dual construction (vLLM ``(vllm_config, role, kv_cache_config)`` or standalone
``(KVConnectorRole.WORKER, req_id=..., transport=..., n_layers=...)``), layer
names ``layer.{i}``, keys ``"{req_id}/layer.{i}/{k|v}"``, bf16/fp16 wire blobs.

Host arrays (numpy, or CPU tensors) take the reference's path unchanged:
ser -> push per layer; pull -> deser -> copy into the registered caches.

CUDA tensors take the device path, with the signatures unchanged:
  save_kv_layer(name, (k, v), num_tokens=P)  k, v CUDA bf16 [T, Hkv, D]
      (token-major, as a prefill produces them): packed on a side stream into
      the S-wide frame, staged through pinned memory and published by one
      ordered writer thread; the files are byte-identical to the host path's.
      save_kv_layer returns at once, so wait_for_save() is a real fence and
      get_finished() reports the request once its files are published.
  register_kv_caches(cache.view(req_id, num_tokens, S))  a PagedRequestView:
      wait_for_layer_load(name) pulls the layer's files into pinned memory,
      copies the payloads to the device and scatters them into the paged cache;
      it returns the layer's device frames (k [Hkv, D, S], v [Hkv, S, D]).
      The load consumes the handoff: once every layer start_load_kv named has
      loaded, the files of those layers are removed from the transport (what
      the reference's decode worker does after its load, serving/cluster.py:
      461-466; a kept request would hold 64 MiB of /dev/shm at S=512). Only
      this request's own keys are removed.

load_request() is that decode-worker load on the host path (serving/cluster.py:
438-467): zeroed float32 K/V, every layer through the connector, then the
request's files removed.
"""
import os
from dataclasses import dataclass, field

import numpy as np

from .kv_base import KVConnectorBase_V1, KVConnectorMetadata, KVConnectorRole
from .transport import InProcTransport, Transport, deser, select_transport, ser  # noqa: F401


@dataclass
class RngdKVConnectorMetadata(KVConnectorMetadata):
    """Scheduler -> worker KV-transfer instructions for one step."""
    req_id: str = ""
    load_layers: list = field(default_factory=list)
    save_layers: list = field(default_factory=list)
    num_external_tokens: int = 0
    remote: str = ""


class RngdKVConnector(KVConnectorBase_V1):
    """KVConnectorBase_V1 implementation for PD disaggregation over a key -> bytes transport."""

    def __init__(self, *args, req_id="r0", transport: Transport = None, n_layers=0,
                 kv_transport=None, frame_tokens=None, **kw):
        if args and isinstance(args[0], KVConnectorRole):
            # standalone: (role, req_id?, transport?, n_layers?) positionally
            role = args[0]
            if len(args) > 1 and isinstance(args[1], str):
                req_id = args[1]
            if len(args) > 2 and args[2] is not None:
                transport = args[2]
            if len(args) > 3:
                n_layers = args[3]
            self._connector_metadata = None
            self._vllm_config = None
            self._kv_transfer_config = None
            self._kv_cache_config = None
            self._role = role
        else:
            vllm_config = args[0] if args else kw.get("vllm_config")
            role = args[1] if len(args) > 1 else kw.get("role")
            kv_cache_config = args[2] if len(args) > 2 else kw.get("kv_cache_config")
            super().__init__(vllm_config, role, kv_cache_config)
            xfer = getattr(self._kv_transfer_config, "kv_connector_extra_config", {}) or {}
            req_id = xfer.get("req_id", req_id)
            n_layers = xfer.get("n_layers", n_layers)
            kv_transport = xfer.get("kv_transport", kv_transport)
            frame_tokens = xfer.get("frame_tokens", frame_tokens)
        self.req_id = req_id
        self.n_layers = n_layers
        self.frame_tokens = frame_tokens
        if transport is None and (kv_transport or os.environ.get("AIRM_KV_TRANSPORT")):
            transport = select_transport(kv_transport)
        self.t = transport or InProcTransport()
        self._kv_caches = None
        self._saved = {}
        self._loading = []
        self._saver = None
        self._loader = None
        self._sent_reqs = set()
        self._loaded = set()

    @property
    def role(self):
        return self._role

    # ---------------- scheduler side ----------------
    def get_num_new_matched_tokens(self, request, num_computed_tokens):
        """(tokens whose KV the prefill side holds beyond what is computed, load async?)."""
        n = getattr(request, "kv_ready_tokens", 0)
        extra = max(0, n - num_computed_tokens)
        return (extra if extra > 0 else None, extra > 0)

    def update_state_after_alloc(self, request, blocks, num_external_tokens):
        self._pending_alloc = (getattr(request, "request_id", self.req_id), num_external_tokens)

    def build_connector_meta(self, scheduler_output):
        layers = [f"layer.{i}" for i in range(self.n_layers)]
        is_worker = self._role == KVConnectorRole.WORKER
        return RngdKVConnectorMetadata(req_id=self.req_id,
                                       save_layers=layers if is_worker else [],
                                       load_layers=layers, num_external_tokens=self.n_layers)

    # ---------------- worker side ----------------
    def register_kv_caches(self, kv_caches):
        """vLLM passes dict[layer_name -> cache]; the standalone runtime passes
        (K_list, V_list) indexed by layer, or a PagedRequestView for the device path."""
        self._kv_caches = kv_caches
        if isinstance(kv_caches, dict) and self.n_layers == 0:
            self.n_layers = len(kv_caches)

    @staticmethod
    def _split_kv(kv_layer):
        """(k, v) host arrays from a (k, v) pair, a stacked [2, ...] array or a CPU tensor."""
        if isinstance(kv_layer, (tuple, list)) and len(kv_layer) == 2:
            k, v = kv_layer
        else:
            arr = kv_layer.detach().cpu().numpy() if hasattr(kv_layer, "detach") else np.asarray(kv_layer)
            if arr.shape[0] != 2:
                raise ValueError(f"expected stacked [2,...] kv_layer, got {arr.shape}")
            k, v = arr[0], arr[1]

        def to_np(x):
            return x.detach().cpu().numpy() if hasattr(x, "detach") else np.asarray(x)
        return to_np(k), to_np(v)

    def save_kv_layer(self, layer_name, kv_layer, attn_metadata=None, **kwargs):
        """Push one layer's KV (prefill side); the device path returns before the write."""
        from .gpu_stage import is_device_tensor, split_device_kv
        first = kv_layer[0] if isinstance(kv_layer, (tuple, list)) else kv_layer
        if is_device_tensor(first):
            k, v = split_device_kv(kv_layer)
            if k.dim() != 3:
                raise ValueError(f"device KV must be token-major [T, Hkv, D], got {tuple(k.shape)}")
            T, H, D = k.shape
            P = int(kwargs.get("num_tokens", T))
            if self._saver is None:
                if getattr(self.t, "device_ipc", False):
                    # Same-GPU consumer: pack into an exported frame slot (no host copy).
                    from .ipc import IpcSaver
                    if not self.n_layers:
                        raise ValueError("the ipc transport needs n_layers to size the frame")
                    pool = self.t.pool(self.n_layers, H, D, self.frame_tokens or T, k.device)
                    self._saver = IpcSaver(self.t, self.req_id, pool)
                else:
                    from .gpu_stage import FrameSaver
                    self._saver = FrameSaver(self.t, self.req_id, H, D, self.frame_tokens or T,
                                             device=k.device)
            self._saver.save(layer_name, k, v, P)
            self._saved[layer_name] = True
            return
        k, v = self._split_kv(kv_layer)
        self.t.push(f"{self.req_id}/{layer_name}/k", ser(k))
        self.t.push(f"{self.req_id}/{layer_name}/v", ser(v))
        self._saved[layer_name] = True

    def wait_for_save(self):
        """Barrier until every pushed layer is published."""
        if self._saver is not None:
            self._saver.wait()
            self._sent_reqs.add(self.req_id)

    def start_load_kv(self, forward_context=None, **kwargs):
        """Begin loading the layers named in the bound metadata (all layers without one)."""
        meta = self._connector_metadata
        self._loading = (list(getattr(meta, "load_layers", [])) if meta
                         else [f"layer.{i}" for i in range(self.n_layers)])

    def wait_for_layer_load(self, layer_name):
        """Block until the layer's KV is present and place it in the registered cache."""
        t = float(os.environ.get("PD_KV_PULL_TIMEOUT", "5"))
        li = int(layer_name.split(".")[-1])
        from ..engines.paged_cache import PagedRequestView
        if isinstance(self._kv_caches, PagedRequestView):
            if self._loader is None:
                view = self._kv_caches
                if getattr(self.t, "device_ipc", False):
                    from .ipc import IpcLoader as Loader
                else:
                    from .gpu_stage import FrameLoader as Loader
                self._loader = Loader(self.t, self.req_id, view, view.cache.n_layers,
                                      view.cache.n_kv_heads, view.cache.head_dim,
                                      device=view.cache.device, timeout=t)
            frames = self._loader.load(layer_name, li)
            self._loaded.add(layer_name)
            self._consume_if_complete()
            return frames
        k = deser(self.t.pull(f"{self.req_id}/{layer_name}/k", timeout=t))
        v = deser(self.t.pull(f"{self.req_id}/{layer_name}/v", timeout=t))
        if self._kv_caches is not None:
            # The producer may ship only the filled columns: place what arrived.
            if isinstance(self._kv_caches, dict):
                dst = self._kv_caches.get(layer_name)
                if dst is not None:
                    dst[0][:] = k
                    dst[1][:] = v
            else:
                self._kv_caches[0][li][:] = k
                self._kv_caches[1][li][:] = v
        return k, v

    def _consume_if_complete(self):
        """Remove the loaded layers' keys once every expected layer is in."""
        expected = set(self._loading or [f"layer.{i}" for i in range(self.n_layers)])
        if not expected or not expected <= self._loaded or getattr(self.t, "device_ipc", False):
            return
        discard = getattr(self.t, "discard", None)
        if discard is None:              # a transport whose pull already consumed (tcp)
            return
        for name in sorted(expected):
            discard(f"{self.req_id}/{name}/k")
            discard(f"{self.req_id}/{name}/v")

    def get_finished(self, finished_req_ids):
        """(requests whose asynchronous save completed, None)."""
        sent, self._sent_reqs = self._sent_reqs, set()
        return (sent or None, None)

    def close(self):
        if self._saver is not None:
            self._saver.close()
            self._saver = None
        if self._loader is not None:
            self._loader.close()
            self._loader = None


def load_request(req_id, n_layers, n_kv_heads, head_dim, S, transport=None):
    """One request's load on the decode side's host path (serving/cluster.py:438-467).

    K [L, Hkv, D, S] and V [L, Hkv, S, D] float32 start at zero (a producer may
    ship only the prompt's columns), every layer is loaded through the
    connector, and the request's files are then removed from the transport.
    Returns (K, V, load_ms)."""
    import time
    K = np.zeros((n_layers, n_kv_heads, head_dim, S), np.float32)
    V = np.zeros((n_layers, n_kv_heads, S, head_dim), np.float32)
    t = transport or select_transport()
    conn = RngdKVConnector(KVConnectorRole.WORKER, req_id=req_id, transport=t, n_layers=n_layers)
    conn.register_kv_caches(([K[i] for i in range(n_layers)], [V[i] for i in range(n_layers)]))
    conn.bind_connector_metadata(conn.build_connector_meta(None))
    t0 = time.perf_counter()
    conn.start_load_kv()
    for i in range(n_layers):
        conn.wait_for_layer_load(f"layer.{i}")
    load_ms = (time.perf_counter() - t0) * 1e3
    if hasattr(t, "discard_request"):
        t.discard_request(req_id)
    elif hasattr(t, "discard"):
        for i in range(n_layers):
            t.discard(f"{req_id}/layer.{i}/k")
            t.discard(f"{req_id}/layer.{i}/v")
    return K, V, load_ms
