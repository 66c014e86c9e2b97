"""Full-size checks at the benchmark configurations, through properties that
do not need the CPU oracle: round trips (scatter . gather = identity on the
touched pages, untouched pages unchanged), token form = page form, zero
delta = bit-exact copy, R(-d) R(d) = identity within rounding, pair norms
preserved, V untouched. Comparisons run on the GPU, one layer at a time."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import bench
from daser_amd import ops, position, workloads

pytestmark = pytest.mark.gpu


def _block_tables(wl):
    tables, k = [], 0
    for n in wl.req_pages:
        tables.append(wl.page_ids[k:k + n].tolist())
        k += n
    return tables


@pytest.mark.parametrize("cfg,dtype", [(2, "bf16"), (4, "fp8")])
def test_round_trip_full_size(gpu, cfg, dtype):
    print(f"case: full-size round trip cfg{cfg}", flush=True)
    wl = workloads.config(cfg)
    full, caches, _ = bench.fill_caches(torch, wl.shape, wl.num_blocks, dtype, gpu, seed=60)
    st = torch.empty(wl.staging_bytes, dtype=torch.uint8, device=gpu)
    ids = torch.from_numpy(wl.page_ids.astype(np.int64)).to(gpu)
    ops.gather(ops.LayerTable(caches), wl.page_ids, wl.slot_offsets, st)
    dst_full = torch.zeros_like(full)
    dst = [dst_full[l] for l in range(wl.shape.num_layers)]
    ops.scatter(ops.LayerTable(dst), wl.page_ids, wl.slot_offsets, st)
    untouched = torch.ones(wl.num_blocks, dtype=torch.bool, device=gpu)
    untouched[ids] = False
    for l in range(wl.shape.num_layers):
        a = caches[l].view(torch.uint8)
        b = dst[l].view(torch.uint8)
        assert torch.equal(a[:, ids], b[:, ids]), f"layer {l}"
        assert not b[:, untouched].any(), f"layer {l}: untouched block written"
    # the record of a random page equals its cache bytes, all layers
    p = len(wl.page_ids) // 3
    o = int(wl.slot_offsets[p])
    rec = st[o:o + wl.shape.slot_bytes].view(wl.shape.num_layers, -1)
    for l in range(wl.shape.num_layers):
        assert torch.equal(rec[l], caches[l][:, int(wl.page_ids[p])].reshape(-1).view(torch.uint8))
    if cfg == 2:  # the slot_mapping form writes the same records
        st2 = torch.zeros_like(st)
        row = wl.shape.num_heads * wl.shape.head_dim * wl.shape.elem_bytes
        sm = ops.slot_mapping_for(_block_tables(wl), wl.req_tokens, wl.shape.block_size)
        ro = ops.token_row_offsets(wl.req_tokens, wl.shape.slot_bytes, wl.shape.block_size, row)
        ops.gather_slots(ops.LayerTable(caches), sm, ro, st2)
        # equal on every valid token row (partial last pages leave tails zero)
        mask = torch.zeros(wl.staging_bytes // row, dtype=torch.bool, device=gpu)
        rows = torch.from_numpy(ro // row).to(gpu)
        lrows = wl.shape.layer_bytes // row
        prow = wl.shape.page_bytes // row
        for l in range(wl.shape.num_layers):
            mask[rows + l * lrows] = True
            mask[rows + l * lrows + prow] = True
        a = st.view(-1, row)
        b = st2.view(-1, row)
        assert torch.equal(a[mask], b[mask])
        assert not b[~mask].any()
    torch.cuda.synchronize()


@pytest.mark.parametrize("cfg", [3, 6])  # 6: one KV head, 4 KiB pages (grouped kernels)
def test_rerotate_full_size_properties(gpu, cfg):
    print(f"case: full-size rerotate cfg{cfg}", flush=True)
    wl = workloads.config(cfg)
    shape = wl.shape
    src_full, src_caches, _ = bench.fill_caches(torch, shape, wl.num_blocks, "bf16", gpu, seed=61)
    # records of every destination page, from the source caches
    st = torch.empty(wl.n_pages * shape.slot_bytes, dtype=torch.uint8, device=gpu)
    offs = wl.slot_offsets
    ops.gather(ops.LayerTable(src_caches), wl.page_ids, offs, st)
    ridx, uniq = position.page_rope_index(wl.chunk_pages, wl.chunk_delta)
    D = shape.head_dim
    fwd = position.delta_tables(uniq, D, 500000.0, device=gpu)
    bwd = position.delta_tables([-d for d in uniq], D, 500000.0, device=gpu)
    ids = torch.from_numpy(wl.page_ids.astype(np.int64)).to(gpu)

    # zero delta everywhere: a bit-exact copy
    d0_full = torch.zeros_like(src_full)
    d0 = [d0_full[l] for l in range(shape.num_layers)]
    ops.scatter_rerotate(ops.LayerTable(d0), wl.page_ids, offs, st, fwd,
                         np.full(wl.n_pages, -1, np.int32))
    for l in range(shape.num_layers):
        assert torch.equal(d0[l][:, ids], src_caches[l][:, ids])
    del d0, d0_full

    # forward by d, back by -d
    mid_full = torch.zeros_like(src_full)
    mid = [mid_full[l] for l in range(shape.num_layers)]
    ops.scatter_rerotate(ops.LayerTable(mid), wl.page_ids, offs, st, fwd, ridx)
    st2 = torch.empty_like(st)
    ops.gather(ops.LayerTable(mid), wl.page_ids, offs, st2)
    back_full = torch.zeros_like(src_full)
    back = [back_full[l] for l in range(shape.num_layers)]
    ops.scatter_rerotate(ops.LayerTable(back), wl.page_ids, offs, st2, bwd, ridx)
    for l in range(shape.num_layers):
        x = src_caches[l][:, ids]
        y = mid[l][:, ids]
        z = back[l][:, ids]
        assert torch.equal(y[1], x[1]) and torch.equal(z[1], x[1]), f"layer {l}: V changed"
        xf, yf, zf = x[0].float(), y[0].float(), z[0].float()
        # pair norms preserved (neox pairs j, j + D/2) within bf16 rounding
        nx = torch.hypot(xf[..., :D // 2], xf[..., D // 2:])
        ny = torch.hypot(yf[..., :D // 2], yf[..., D // 2:])
        assert ((ny - nx).abs() <= 2 ** -7 * nx + 1e-6).all(), f"layer {l}: norm"
        # round trip: two bf16 roundings, relative to the row's magnitude
        rowmax = xf.abs().amax(dim=-1, keepdim=True)
        assert ((zf - xf).abs() <= 2 ** -7 * rowmax).all(), f"layer {l}: inverse"
        assert (yf != xf).float().mean() > 0.5, f"layer {l}: K was not rotated"
    torch.cuda.synchronize()


@pytest.mark.parametrize("cfg", [3, 6])
def test_split_x_rerotate_equals_token_major_full_size(gpu, cfg):
    """At full size, re-rotating split-x pages (vLLM's PagedAttention K
    layout) gives exactly the bits of re-rotating the same data in token-major
    pages, after the layout permutation: the two entry points run the same
    arithmetic per element (the token-major path is pinned to the oracle)."""
    print(f"case: full-size split-x re-rotate cfg{cfg}", flush=True)
    wl = workloads.config(cfg)
    shape = wl.shape
    L, bs, H, D = shape.num_layers, shape.block_size, shape.num_heads, shape.head_dim
    X = 16 // shape.elem_bytes
    src_full, src_caches, _ = bench.fill_caches(torch, shape, wl.num_blocks, "bf16", gpu, seed=62)
    n = wl.n_pages
    st = torch.empty(n * shape.slot_bytes, dtype=torch.uint8, device=gpu)
    ops.gather(ops.LayerTable(src_caches), wl.page_ids, wl.slot_offsets, st)
    del src_caches, src_full
    ridx, uniq = position.page_rope_index(wl.chunk_pages, wl.chunk_delta)
    fwd = position.delta_tables(uniq, D, 500000.0, device=gpu)
    ids = torch.from_numpy(wl.page_ids.astype(np.int64)).to(gpu)

    nhd_full = torch.zeros((L, 2, wl.num_blocks, bs, H, D), dtype=torch.bfloat16, device=gpu)
    ops.scatter_rerotate(ops.LayerTable([nhd_full[l] for l in range(L)]), wl.page_ids,
                         wl.slot_offsets, st, fwd, ridx)
    # the same records with every page in split-x order
    st_kx = (st.view(torch.bfloat16).view(n, L, 2, bs, H, D // X, X)
             .permute(0, 1, 2, 4, 5, 3, 6).contiguous().view(-1).view(torch.uint8))
    del st
    kx_full = torch.zeros((L, 2, wl.num_blocks, bs * H * D), dtype=torch.bfloat16, device=gpu)
    ops.scatter_rerotate(ops.LayerTable([kx_full[l] for l in range(L)], block_size=bs,
                                        head_dim=D),
                         wl.page_ids, wl.slot_offsets, st_kx, fwd, ridx)
    for l in range(L):
        a = nhd_full[l][:, ids]
        b = (kx_full[l][:, ids].view(2, n, H, D // X, bs, X)
             .permute(0, 1, 4, 2, 3, 5).reshape(2, n, bs, H, D))
        assert torch.equal(a.view(torch.int16), b.view(torch.int16)), f"layer {l}"
    torch.cuda.synchronize()
