"""PagedKVLayout on the CPU (shapes and strides only): which vLLM cache
layouts are accepted, and the geometry each yields."""

from __future__ import annotations

import pytest
import torch

from daser_amd.ops import PagedKVLayout


def _hnd(nb, bs, h, d):
    """(2, NB, bs, H, D) view of head-major memory (2, NB, H, bs, D)."""
    return torch.zeros((2, nb, h, bs, d), dtype=torch.bfloat16).permute(0, 1, 3, 2, 4)


def test_token_major_5d():
    lay = PagedKVLayout.from_caches([torch.zeros((2, 10, 16, 8, 128), dtype=torch.bfloat16)] * 3)
    assert (lay.block_size, lay.num_heads, lay.head_dim, lay.k_layout) == (16, 8, 128, "nhd")
    assert lay.page_bytes == 16 * 8 * 128 * 2 and lay.layer_bytes == 2 * lay.page_bytes
    assert lay.slot_bytes == 3 * lay.layer_bytes and lay.has_geometry


def test_block_major_allocation_viewed_kv_first():
    t = torch.zeros((10, 2, 16, 8, 128), dtype=torch.bfloat16).transpose(0, 1)
    lay = PagedKVLayout.from_caches([t])
    assert lay.kv_stride == 16 * 8 * 128 * 2 and lay.page_stride == 2 * lay.kv_stride


def test_head_major_pages():
    lay = PagedKVLayout.from_caches([_hnd(10, 16, 8, 128)])
    assert (lay.k_layout, lay.block_size, lay.num_heads, lay.head_dim) == ("hnd", 16, 8, 128)
    assert lay.page_bytes == 16 * 8 * 128 * 2
    with pytest.raises(ValueError):
        PagedKVLayout.from_caches([_hnd(10, 16, 8, 128)], k_layout="nhd")
    # one KV head: head-major and token-major memory coincide
    lay = PagedKVLayout.from_caches([_hnd(10, 16, 1, 128)])
    assert lay.k_layout == "nhd" and lay.page_bytes == 16 * 128 * 2
    # a page that is not contiguous in memory at all
    sliced = torch.zeros((2, 10, 16, 8, 256), dtype=torch.bfloat16)[..., :128]
    with pytest.raises(ValueError, match="contiguous"):
        PagedKVLayout.from_caches([sliced])


def test_flat_paged_attention_caches():
    t = torch.zeros((2, 10, 16 * 8 * 128), dtype=torch.float16)
    assert not PagedKVLayout.from_caches([t]).has_geometry  # copies only
    lay = PagedKVLayout.from_caches([t], block_size=16, head_dim=128)
    assert (lay.num_heads, lay.k_layout, lay.has_geometry) == (8, "kx", True)
    with pytest.raises(ValueError):
        PagedKVLayout.from_caches([t], block_size=16, head_dim=96)  # not a whole page
    with pytest.raises(ValueError):
        PagedKVLayout.from_caches([t], block_size=16, head_dim=128, k_layout="hnd")


def test_five_d_geometry_must_agree():
    t = torch.zeros((2, 10, 16, 8, 128), dtype=torch.bfloat16)
    with pytest.raises(ValueError):
        PagedKVLayout.from_caches([t], block_size=32)
    with pytest.raises(ValueError):
        PagedKVLayout.from_caches([t], k_layout="kx")


def test_mismatched_layers_and_bad_ranks():
    a = torch.zeros((2, 10, 16, 8, 128), dtype=torch.bfloat16)
    with pytest.raises(ValueError):
        PagedKVLayout.from_caches([a, torch.zeros((2, 10, 16, 8, 64), dtype=torch.bfloat16)])
    with pytest.raises(ValueError):
        PagedKVLayout.from_caches([torch.zeros((10, 4096), dtype=torch.bfloat16)])
    with pytest.raises(ValueError):
        PagedKVLayout.from_caches([])
