"""DaserConfig.resolved_slot_size against the reference's tests and
constants (tests/test_config.py:7-27, tests/integration/conftest.py:26-30,
benchmarks/bench_storage_imdb.py:45-48), and against the layout the kernels
derive from the caches."""

import pytest
import torch

from daser_amd.config import DaserConfig
from daser_amd.ops import PagedKVLayout


def test_explicit_slot_size():
    assert DaserConfig(slot_size=1024).resolved_slot_size() == 1024


@pytest.mark.parametrize("layers,dtype_bytes,expected", [
    (28, 2, 8 * 128 * 2 * 28 * 16 * 2),
    (36, 2, 2_359_296),
    (32, 2, 2_097_152),
    (32, 1, 1_048_576),  # e4m3 KV
])
def test_computed_slot_size(layers, dtype_bytes, expected):
    cfg = DaserConfig(num_kv_heads=8, head_dim=128, num_layers=layers, dtype_bytes=dtype_bytes)
    assert cfg.resolved_slot_size() == expected
    dt = torch.bfloat16 if dtype_bytes == 2 else torch.float8_e4m3fn
    caches = [torch.empty((2, 4, 16, 8, 128), dtype=dt, device="meta") for _ in range(layers)]
    assert PagedKVLayout.from_caches(caches).slot_bytes == expected


def test_missing_model_param_raises():
    with pytest.raises(ValueError, match="num_layers"):
        DaserConfig(num_kv_heads=8, head_dim=128).resolved_slot_size()
