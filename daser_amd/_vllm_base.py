"""Stand-ins for vLLM's connector base types, used only when vLLM is not
installed (tests, benchmarks). They carry exactly the surface the DaseR
connector relies on: the role enum, the metadata base class, and the base
connector's metadata binding (vllm.distributed.kv_transfer.kv_connector.v1
.base, as called by the reference daser/connector/daser_connector.py:139-141,
:440, :452, :692)."""

from __future__ import annotations

import enum
from typing import Any, Optional


class KVConnectorRole(enum.Enum):
    SCHEDULER = 0
    WORKER = 1


class KVConnectorMetadata:
    """Base of the per-step scheduler -> worker metadata."""


class KVConnectorBase_V1:
    def __init__(self, vllm_config: Any, role: KVConnectorRole, kv_cache_config: Any = None) -> None:
        self._vllm_config = vllm_config
        self._role = role
        self._kv_cache_config = kv_cache_config
        self._connector_metadata: Optional[KVConnectorMetadata] = None

    @property
    def role(self) -> KVConnectorRole:
        return self._role

    def bind_connector_metadata(self, connector_metadata: KVConnectorMetadata) -> None:
        self._connector_metadata = connector_metadata

    def clear_connector_metadata(self) -> None:
        self._connector_metadata = None

    def has_connector_metadata(self) -> bool:
        return self._connector_metadata is not None

    def _get_connector_metadata(self) -> KVConnectorMetadata:
        assert self._connector_metadata is not None
        return self._connector_metadata
