"""DaseR configuration (reference daser/config.py:8-75).

Only ``resolved_slot_size`` touches the data path: the bytes of one block's
record over all layers, which the connector derives from the registered
caches and the server uses for file offsets (start_slot * slot_size).
"""

from __future__ import annotations

from dataclasses import dataclass


@dataclass
class DaserConfig:
    store_path: str = "/mnt/xfs/daser.store"
    index_path: str = "/mnt/xfs/daser.index"
    total_slots: int = 1024
    slot_size: int = 0
    ipc_socket_path: str = "/tmp/daser.sock"
    log_level: str = "INFO"
    perf_log_enabled: bool = False
    num_kv_heads: int = 0
    head_dim: int = 0
    num_layers: int = 0
    block_tokens: int = 16
    dtype_bytes: int = 2
    model_id: str = "default"

    def resolved_slot_size(self) -> int:
        """slot_size if set, else num_kv_heads * head_dim * 2 (K and V) *
        num_layers * block_tokens * dtype_bytes; raises ValueError naming the
        first missing model parameter (reference :47-75)."""
        if self.slot_size > 0:
            return self.slot_size
        for value, name in ((self.num_kv_heads, "num_kv_heads"), (self.head_dim, "head_dim"),
                            (self.num_layers, "num_layers")):
            if value == 0:
                raise ValueError(f"slot_size is 0 but {name} is also 0; "
                                 "provide either slot_size or all model params")
        return (self.num_kv_heads * self.head_dim * 2 * self.num_layers * self.block_tokens
                * self.dtype_bytes)
