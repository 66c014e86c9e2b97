"""dsr_scatter_rerotate_static (host tables staged in the library's fixed
device array, no allocation) writes the same bytes as dsr_scatter_rerotate
(device tables), called through the C ABI: two calls in a row on one
stream, the second with fewer pages, so the second call's staged tables
overwrite the first's."""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from daser_amd import _lib
from daser_amd.workloads import KVShape
from tests.helpers import rand_caches

pytestmark = pytest.mark.gpu

SHAPE = KVShape(4, 8, 128, 16, 2)  # L4 H8 D128 bs16, Llama-3-8B rows
NB = 256


def _cos_sin(n_groups, n_tables, half, seed):
    rng = np.random.default_rng(seed)
    ang = rng.uniform(-4000.0, 4000.0, (n_groups, n_tables, 1)) * \
        (500000.0 ** (-np.arange(half) / half))[None, None, :]
    return np.stack([np.cos(ang), np.sin(ang)], -1).astype(np.float32)


def _ptr(a: np.ndarray):
    return ctypes.c_void_p(a.ctypes.data)


@pytest.mark.parametrize("dt", ["bf16", "e4m3"])
def test_static_matches_device_table_entry_point(dt):
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    L, bs, H, D = SHAPE.num_layers, SHAPE.block_size, SHAPE.num_heads, SHAPE.head_dim
    esize = 2 if dt == "bf16" else 1
    dcode = _lib.DSR_DTYPE_BF16 if dt == "bf16" else _lib.DSR_DTYPE_FP8_E4M3
    page_bytes = bs * H * D * esize
    layer_bytes = 2 * page_bytes
    slot = L * layer_bytes
    rng = np.random.default_rng(7)
    n_rec = 200
    staging = torch.from_numpy(rng.integers(0, 256, n_rec * slot, dtype=np.uint8))
    if dt == "e4m3":  # no NaN codes in the records: NaN bytes are compared as bytes anyway
        staging[(staging & 0x7F) == 0x7F] = 0x10
    staging = staging.to(dev)
    caches_a = rand_caches(SHAPE, NB, dt, dev, seed=3)
    caches_b = [c.clone() for c in caches_a]
    kv_stride = caches_a[0].stride(0) * esize
    page_stride = caches_a[0].stride(1) * esize
    half = D // 2
    lib = _lib.lib()
    stream = torch.cuda.current_stream(dev).cuda_stream
    # per-layer groups (layer 2 has no RoPE) and scales
    n_groups, n_tables = 2, 6
    cos_sin = _cos_sin(n_groups, n_tables, half, seed=11)
    layer_group = np.array([0, 1, -1, 0], dtype=np.int32)
    k_scale = np.array([0.02, 0.05, 0.03, 0.011], dtype=np.float32) if dt == "e4m3" else None
    cos_sin_d = torch.from_numpy(cos_sin).to(dev)
    lg_d = torch.from_numpy(layer_group).to(dev)
    ks_d = torch.from_numpy(k_scale).to(dev) if k_scale is not None else None

    for n_pages, seed in ((n_rec, 1), (57, 2)):
        r = np.random.default_rng(seed)
        page_ids = r.permutation(NB)[:n_pages].astype(np.int32)
        slot_offsets = (r.permutation(n_rec)[:n_pages].astype(np.int64) * slot)
        rope_idx = r.integers(-1, n_tables, n_pages).astype(np.int32)
        bases_a = np.array([c.data_ptr() for c in caches_a], dtype=np.uint64)
        bases_b = np.array([c.data_ptr() for c in caches_b], dtype=np.uint64)
        print(f"static scatter_rerotate dt={dt} n_pages={n_pages}", flush=True)
        # existing entry point: device tables
        t = [torch.from_numpy(x).to(dev) for x in (bases_a, page_ids, slot_offsets, rope_idx)]
        rc = lib.dsr_scatter_rerotate(
            t[0].data_ptr(), L, kv_stride, page_stride, page_bytes, NB, t[1].data_ptr(),
            t[2].data_ptr(), n_pages, staging.data_ptr(), staging.numel(), layer_bytes, 0,
            cos_sin_d.data_ptr(), t[3].data_ptr(), n_tables, lg_d.data_ptr(), n_groups, D, D,
            _lib.DSR_ROPE_NEOX, dcode, None if ks_d is None else ks_d.data_ptr(), 0, stream)
        _lib.check("dsr_scatter_rerotate", rc)
        # allocation-free entry point: host tables
        rc = lib.dsr_scatter_rerotate_static(
            _ptr(bases_b), L, kv_stride, page_stride, page_bytes, NB, _ptr(page_ids),
            _ptr(slot_offsets), n_pages, staging.data_ptr(), staging.numel(), layer_bytes, 0,
            _ptr(cos_sin), _ptr(rope_idx), n_tables, _ptr(layer_group), n_groups, D, D,
            _lib.DSR_ROPE_NEOX, dcode, None if k_scale is None else _ptr(k_scale), 0, stream)
        _lib.check("dsr_scatter_rerotate_static", rc)
        torch.cuda.synchronize(dev)
        for l in range(L):
            a = caches_a[l].view(torch.uint8)
            b = caches_b[l].view(torch.uint8)
            assert torch.equal(a, b), (dt, n_pages, l)
        # the loaded pages really changed (the call did work)
        rec = staging.view(n_rec, L, 2, page_bytes)
        v_got = caches_b[3].view(torch.uint8)[1, torch.from_numpy(page_ids).long().to(dev)]
        v_want = rec[torch.from_numpy(slot_offsets // slot).to(dev), 3, 1]
        assert torch.equal(v_got.reshape(n_pages, -1), v_want)

