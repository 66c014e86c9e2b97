"""Full-size checks at the benchmark configurations (2-6, the sizes bench.py
times), two ways:

* oracle samples: after each full-size launch, 64 seeded pages (every
  layer) are copied to the host and compared with the CPU oracle run on the
  same pages' inputs: bit-exact for gather/scatter bytes and V, within the
  re-rotation tolerance for K (oracle.rotation_within_tolerance);
* properties over every page: round trips (scatter . gather = identity on
  the touched pages, untouched pages unchanged), token form = page form,
  zero delta = bit-exact copy, R(-d) R(d) = identity within rounding, pair
  norms preserved, V untouched. Comparisons run on the GPU, one layer at a
  time."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import bench
from daser_amd import ops, position, workloads
from oracle import oracle

pytestmark = pytest.mark.gpu

N_SAMPLE = 64
THETA = 500000.0


def _sample(n_pages: int, seed: int) -> np.ndarray:
    rng = np.random.default_rng(seed)
    return np.sort(rng.choice(n_pages, size=min(N_SAMPLE, n_pages), replace=False))


def _host_bits(t: torch.Tensor) -> np.ndarray:
    """Raw element bits of a device tensor on the host (uint16 or uint8)."""
    if t.element_size() == 2:
        return t.cpu().view(torch.int16).numpy().view(np.uint16)
    return t.cpu().view(torch.uint8).numpy()


def _records(staging: torch.Tensor, offsets, slot_bytes: int) -> np.ndarray:
    """The slot records at ``offsets``, back to back, on the host."""
    return torch.cat([staging[int(o):int(o) + slot_bytes] for o in offsets]).cpu().numpy()


def _cache_pages(caches, blocks) -> list[np.ndarray]:
    """Per layer, the (2, n, bs, H, D) pages of ``blocks`` on the host."""
    ids = torch.from_numpy(np.asarray(blocks, np.int64)).to(caches[0].device)
    return [np.ascontiguousarray(_host_bits(c[:, ids])) for c in caches]


def check_gather_sample(wl, caches, staging, seed):
    """The kernel's records of sampled pages = oracle.gather of those pages."""
    sh = wl.shape
    sel = _sample(wl.n_pages, seed)
    pages = _cache_pages(caches, wl.page_ids[sel])
    want = np.zeros(sel.size * sh.slot_bytes, np.uint8)
    oracle.gather(pages, np.arange(sel.size), np.arange(sel.size) * sh.slot_bytes, want,
                  sh.layer_bytes)
    got = _records(staging, wl.slot_offsets[sel], sh.slot_bytes)
    assert np.array_equal(got, want), "gather records differ from the oracle"


def check_scatter_sample(wl, caches, staging, src_offsets, seed):
    """The kernel's cache pages of sampled pages = oracle.scatter of their records."""
    sh = wl.shape
    sel = _sample(wl.n_pages, seed)
    recs = _records(staging, src_offsets[sel], sh.slot_bytes)
    dt = np.uint16 if sh.elem_bytes == 2 else np.uint8
    want = [np.zeros((2, sel.size, sh.block_size, sh.num_heads, sh.head_dim), dt)
            for _ in range(sh.num_layers)]
    oracle.scatter(want, np.arange(sel.size), np.arange(sel.size) * sh.slot_bytes, recs,
                   sh.layer_bytes)
    got = _cache_pages(caches, wl.page_ids[sel])
    for l in range(sh.num_layers):
        assert np.array_equal(got[l], want[l]), f"layer {l}: scatter differs from the oracle"


def check_rerotate_sample(wl, caches, staging, src_offsets, page_delta, dtype, seed,
                          k_scale=None):
    """Sampled pages of a full-size re-rotating scatter against
    oracle.scatter_rerotate on the same records: V bit-exact, K within 1 ulp
    of the float64 rotation (cancellation-aware)."""
    sh = wl.shape
    sel = _sample(wl.n_pages, seed)
    recs = _records(staging, src_offsets[sel], sh.slot_bytes)
    dt = np.uint16 if sh.elem_bytes == 2 else np.uint8
    want = [np.zeros((2, sel.size, sh.block_size, sh.num_heads, sh.head_dim), dt)
            for _ in range(sh.num_layers)]
    ks = None if k_scale is None else k_scale.detach().cpu().numpy().astype(np.float32)
    oracle.scatter_rerotate(want, np.arange(sel.size), np.arange(sel.size) * sh.slot_bytes,
                            recs, sh.layer_bytes, dtype=dtype, rot_dim=sh.head_dim,
                            style=oracle.NEOX, stored_pos=np.zeros(sel.size, np.int64),
                            new_pos=np.asarray(page_delta, np.int64)[sel],
                            rotate=np.ones(sel.size, np.int8), theta=THETA, k_scale=ks)
    got = _cache_pages(caches, wl.page_ids[sel])
    stored = recs.view(dt).reshape(sel.size, sh.num_layers, 2, sh.block_size, sh.num_heads,
                                   sh.head_dim)
    moved = 0
    for l in range(sh.num_layers):
        assert np.array_equal(got[l][1], want[l][1]), f"layer {l}: V differs from the oracle"
        ok, msg = oracle.rotation_within_tolerance(got[l][0], want[l][0], dtype)
        assert ok, f"layer {l}: K outside tolerance: {msg}"
        moved += int((got[l][0] != stored[:, l, 0]).sum())
    assert moved > 0, "no K element was rotated"


def check_slots_rerotate_sample(wl, caches, staging, sm, ro, tok_delta, seed, n_tok=256):
    """Sampled tokens of a full-size token-form re-rotating scatter against
    oracle.scatter_slots_rerotate run on just those tokens: their record
    rows (all layers) are packed into a small host staging and their
    destination slots into a small host pool. V rows bit-exact, K within the
    rotation tolerance."""
    sh = wl.shape
    bs, row = sh.block_size, sh.num_heads * sh.head_dim * sh.elem_bytes
    rng = np.random.default_rng(seed)
    valid = np.flatnonzero(sm >= 0)
    sel = np.sort(rng.choice(valid, size=min(n_tok, valid.size), replace=False))
    n = sel.size
    # token i of the sample: host record row (i // bs, row i % bs) and host
    # slot i (block i // bs, offset i % bs)
    ro_h = (np.arange(n) // bs) * sh.slot_bytes + (np.arange(n) % bs) * row
    rows = staging.view(-1, row)
    lrows, prow = sh.layer_bytes // row, sh.page_bytes // row
    src_rows = torch.from_numpy(ro[sel] // row).to(staging.device)
    n_slots = -(-n // bs)
    recs = torch.zeros(n_slots * sh.slot_bytes, dtype=torch.uint8, device=staging.device)
    dst_rows = torch.from_numpy(ro_h // row).to(staging.device)
    rrows = recs.view(-1, row)
    for l in range(sh.num_layers):
        for half in (0, prow):
            rrows[dst_rows + l * lrows + half] = rows[src_rows + l * lrows + half]
    dt = np.uint16 if sh.elem_bytes == 2 else np.uint8
    want = [np.zeros((2, n_slots, bs, sh.num_heads, sh.head_dim), dt)
            for _ in range(sh.num_layers)]
    d = np.asarray(tok_delta, np.int64)[sel]
    oracle.scatter_slots_rerotate(
        want, np.arange(n, dtype=np.int64), ro_h, recs.cpu().numpy(), sh.layer_bytes,
        dtype=oracle.BF16 if sh.elem_bytes == 2 else oracle.E4M3, rot_dim=sh.head_dim,
        style=oracle.NEOX, stored_pos=np.zeros(n, np.int64), new_pos=d, rotate=d != 0,
        theta=THETA)
    blk = torch.from_numpy(sm[sel] // bs).to(staging.device)
    off = torch.from_numpy(sm[sel] % bs).to(staging.device)
    for l in range(sh.num_layers):
        got = _host_bits(caches[l][:, blk, off])  # (2, n, H, D)
        w = want[l].reshape(2, n_slots * bs, sh.num_heads, sh.head_dim)[:, :n]
        assert np.array_equal(got[1], w[1]), f"layer {l}: V differs from the oracle"
        assert got[1].any(), f"layer {l}: sampled rows are empty"
        ok, msg = oracle.rotation_within_tolerance(got[0], w[0], oracle.BF16)
        assert ok, f"layer {l}: K outside tolerance: {msg}"


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
    check_gather_sample(wl, caches, st, seed=cfg)
    dst_full = torch.zeros_like(full)
    dst = [dst_full[l] for l in range(wl.shape.num_layers)]
    ops.scatter(ops.LayerTable(dst), wl.page_ids, wl.slot_offsets, st)
    check_scatter_sample(wl, dst, st, wl.slot_offsets, seed=cfg + 100)
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
        # the token-form load with every request re-rotated, sampled
        rng = np.random.default_rng(9)
        req_delta = rng.integers(1, 32768, size=len(wl.req_tokens))
        tok_delta = np.repeat(req_delta, wl.req_tokens)
        uniq = sorted(set(int(x) for x in req_delta))
        ridx = np.searchsorted(np.asarray(uniq), tok_delta)
        tabs = position.delta_tables(uniq, wl.shape.head_dim, THETA, device=gpu)
        dst_full.zero_()
        ops.scatter_slots_rerotate(ops.LayerTable(dst), sm, ro, st2, tabs, ridx)
        check_slots_rerotate_sample(wl, dst, st2, sm, ro, tok_delta, seed=21)
    torch.cuda.synchronize()
    del full, caches, dst_full, dst, st
    torch.cuda.empty_cache()


@pytest.mark.parametrize("cfg", [3, 5, 6])
def test_rerotate_full_size_oracle_sample(gpu, cfg):
    """The benchmark's re-rotating scatter at full size (config 5: 80 layers,
    171.8 GB of destination caches, 64 shared source chunks read by many
    pages: host tables with shared records take the fan-out load, each
    record read once), sampled against the oracle."""
    print(f"case: full-size rerotate oracle sample cfg{cfg}", flush=True)
    wl = workloads.config(cfg)
    sh = wl.shape
    src_bytes = wl.meta["src_staging_bytes"]
    src = torch.empty(src_bytes, dtype=torch.uint8, device=gpu)
    g = torch.Generator(device=gpu).manual_seed(70 + cfg)
    for i in range(0, src_bytes, 1 << 30):
        src[i:i + min(1 << 30, src_bytes - i)].view(torch.bfloat16).normal_(generator=g)
    full = torch.empty((sh.num_layers, 2, wl.num_blocks, sh.block_size, sh.num_heads,
                        sh.head_dim), dtype=torch.bfloat16, device=gpu)
    caches = [full[l] for l in range(sh.num_layers)]
    ridx, uniq = position.page_rope_index(wl.chunk_pages, wl.chunk_delta)
    tabs = position.delta_tables(uniq, sh.head_dim, THETA, device=gpu)
    shared = bool(2 * np.unique(wl.src_offsets).size <= wl.src_offsets.size)
    assert shared == (cfg != 3)
    ops.scatter_rerotate(ops.LayerTable(caches), wl.page_ids, wl.src_offsets, src, tabs, ridx)
    torch.cuda.synchronize()
    check_rerotate_sample(wl, caches, src, wl.src_offsets, wl.page_delta, oracle.BF16,
                          seed=200 + cfg)
    del full, caches, src
    torch.cuda.empty_cache()


def test_fp8_rerotate_full_size_oracle_sample(gpu):
    """Config 4's e4m3 re-rotation at full size (128 requests, 1.09 M tokens,
    per-layer fp32 K scales, every request moved by its own delta), sampled
    against the oracle's dequantise -> rotate -> requantise."""
    print("case: full-size fp8 rerotate oracle sample cfg4", flush=True)
    wl = workloads.config(4)
    sh = wl.shape
    full, caches, k_scale = bench.fill_caches(torch, sh, wl.num_blocks, "fp8", gpu, seed=64)
    st = torch.empty(wl.staging_bytes, dtype=torch.uint8, device=gpu)
    ops.gather(ops.LayerTable(caches), wl.page_ids, wl.slot_offsets, st)
    del full, caches
    rng = np.random.default_rng(7)
    deltas = rng.integers(1, 32768, size=len(wl.req_pages)).tolist()
    ridx, uniq = position.page_rope_index(wl.req_pages, deltas)
    tabs = position.delta_tables(uniq, sh.head_dim, THETA, device=gpu)
    dst_full = torch.empty((sh.num_layers, 2, wl.num_blocks, sh.block_size, sh.num_heads,
                            sh.head_dim), dtype=torch.float8_e4m3fn, device=gpu)
    dst = [dst_full[l] for l in range(sh.num_layers)]
    ops.scatter_rerotate(ops.LayerTable(dst), wl.page_ids, wl.slot_offsets, st, tabs, ridx,
                         k_scale=k_scale)
    torch.cuda.synchronize()
    page_delta = np.repeat(np.asarray(deltas, np.int64), wl.req_pages)
    check_rerotate_sample(wl, dst, st, wl.slot_offsets, page_delta, oracle.E4M3, seed=204,
                          k_scale=k_scale)
    del dst_full, dst, st
    torch.cuda.empty_cache()


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
