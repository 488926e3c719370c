"""vLLM's KVConnector v1 base types, or a local stand-in with the same surface.

With vLLM 0.18.0 importable the real ``KVConnectorBase_V1``, ``KVConnectorRole``
and ``KVConnectorMetadata`` are used, so ``isinstance(conn, KVConnectorBase_V1)``
holds for the engine. Without it, the stand-in below provides the part of the
base class the connector relies on: the role enum, the metadata base class and
bind/clear/get of the per-step connector metadata (the reference's standalone
construction replicates exactly this state, connector/rngd_kv.py:49-54).
"""
import enum

try:  # pragma: no cover - exercised only where vLLM is installed
    from vllm.distributed.kv_transfer.kv_connector.v1.base import (  # noqa: F401
        KVConnectorBase_V1, KVConnectorMetadata, KVConnectorRole)
    HAVE_VLLM = True
except ImportError:
    HAVE_VLLM = False

if not HAVE_VLLM:

    class KVConnectorRole(enum.Enum):
        SCHEDULER = 0
        WORKER = 1

    class KVConnectorMetadata:
        """Per-step scheduler -> worker instructions (subclassed by connectors)."""

    class KVConnectorBase_V1:
        """The v1 connector surface: scheduler-side and worker-side hooks."""

        def __init__(self, vllm_config=None, role=KVConnectorRole.WORKER, kv_cache_config=None):
            self._connector_metadata = None
            self._vllm_config = vllm_config
            self._kv_transfer_config = getattr(vllm_config, "kv_transfer_config", None)
            self._kv_cache_config = kv_cache_config
            self._role = role

        @property
        def role(self):
            return self._role

        def bind_connector_metadata(self, connector_metadata):
            self._connector_metadata = connector_metadata

        def clear_connector_metadata(self):
            self._connector_metadata = None

        def _get_connector_metadata(self):
            if self._connector_metadata is None:
                raise AssertionError("connector metadata is not bound")
            return self._connector_metadata

        # worker side
        def register_kv_caches(self, kv_caches):
            pass

        def start_load_kv(self, forward_context, **kwargs):
            raise NotImplementedError

        def wait_for_layer_load(self, layer_name):
            raise NotImplementedError

        def save_kv_layer(self, layer_name, kv_layer, attn_metadata, **kwargs):
            raise NotImplementedError

        def wait_for_save(self):
            raise NotImplementedError

        def get_finished(self, finished_req_ids):
            return None, None

        # scheduler side
        def get_num_new_matched_tokens(self, request, num_computed_tokens):
            raise NotImplementedError

        def update_state_after_alloc(self, request, blocks, num_external_tokens):
            raise NotImplementedError

        def build_connector_meta(self, scheduler_output):
            raise NotImplementedError
