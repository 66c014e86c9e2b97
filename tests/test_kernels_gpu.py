"""Parity of the HIP kernels against the C oracle (bit-exact copies, <= 1 ulp
re-rotation), called through the C ABI via daser_amd.ops."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from daser_amd import ops, position, workloads
from daser_amd._lib import DaserKVError
from daser_amd.workloads import KVShape
from oracle import oracle
from tests.helpers import ORC_DT, rand_caches, rotation_within_tolerance, to_bits_np

pytestmark = pytest.mark.gpu

FP8 = ("e4m3", "e5m2")


def _np_layers(caches, dt):
    return [to_bits_np(c, dt) for c in caches]


def _gather_both(wl, caches, dt, gpu):
    table = ops.LayerTable(caches)
    staging = torch.zeros(wl.staging_bytes, dtype=torch.uint8, device=gpu)
    ops.gather(table, wl.page_ids, wl.slot_offsets, staging)
    ref = np.zeros(wl.staging_bytes, dtype=np.uint8)
    oracle.gather(_np_layers(caches, dt), wl.page_ids, wl.slot_offsets, ref,
                  wl.shape.layer_bytes)
    return staging, ref


def test_gather_cfg1_bit_exact(gpu):
    print("case: gather cfg1", flush=True)
    wl = workloads.config(1)
    caches = rand_caches(wl.shape, wl.num_blocks, "bf16", gpu, seed=1)
    staging, ref = _gather_both(wl, caches, "bf16", gpu)
    torch.cuda.synchronize()
    assert np.array_equal(staging.cpu().numpy(), ref)


def test_scatter_cfg1_bit_exact_and_round_trip(gpu):
    print("case: scatter cfg1", flush=True)
    wl = workloads.config(1)
    caches = rand_caches(wl.shape, wl.num_blocks, "bf16", gpu, seed=2)
    staging, ref = _gather_both(wl, caches, "bf16", gpu)
    dst = [torch.zeros_like(c) for c in caches]
    ops.scatter(ops.LayerTable(dst), wl.page_ids, wl.slot_offsets, staging)
    dst_ref = [np.zeros_like(a) for a in _np_layers(caches, "bf16")]
    oracle.scatter(dst_ref, wl.page_ids, wl.slot_offsets, ref, wl.shape.layer_bytes)
    torch.cuda.synchronize()
    touched = torch.zeros(wl.num_blocks, dtype=torch.bool)
    touched[torch.from_numpy(wl.page_ids.astype(np.int64))] = True
    for l in range(wl.shape.num_layers):
        got = to_bits_np(dst[l], "bf16")
        assert np.array_equal(got, dst_ref[l])
        # scatter . gather = identity on touched pages, untouched stay zero
        assert torch.equal(dst[l][:, touched.to(gpu)], caches[l][:, touched.to(gpu)])
        assert not dst[l][:, (~touched).to(gpu)].view(torch.int16).any()


@pytest.mark.parametrize("heads,head_dim,dt", [(8, 128, "bf16"), (16, 128, "bf16"),
                                                (8, 128, "e4m3"), (4, 96, "bf16")])
@pytest.mark.parametrize("kernel,wg_per_cu", [(0, 0), (1, 0), (2, 0), (1, 1), (2, 1), (2, 2),
                                              (3, 1), (3, 2), (1, 3)])
def test_page_copy_kernels_and_occupancy_match_oracle(gpu, tuning, heads, head_dim, dt,
                                                      kernel, wg_per_cu):
    """Both one-unit scatter kernels (load-all-then-store, streaming in
    either unit order) at every occupancy the launch policy or an override may pick, and the
    gather at the same occupancies: the oracle's bytes, with ragged requests
    and partial last pages (pages of 32, 64, 16 and 12 KiB)."""
    print(f"case: page copy H{heads} D{head_dim} {dt} kernel={kernel} wpc={wg_per_cu}",
          flush=True)
    tuning("scatter_kernel", kernel)
    tuning("copy_wg_per_cu", wg_per_cu)
    shape = KVShape(3, heads, head_dim, 16, 1 if dt in FP8 else 2)
    wl = workloads.ragged(shape, 6, 1, 400, seed=heads + head_dim, pool_slack=1.3)
    caches = rand_caches(shape, wl.num_blocks, dt, gpu, seed=9, scale=3.0)
    staging, ref = _gather_both(wl, caches, dt, gpu)
    torch.cuda.synchronize()
    assert np.array_equal(staging.cpu().numpy(), ref)
    dst = rand_caches(shape, wl.num_blocks, dt, gpu, seed=10)
    dst_ref = _np_layers(dst, dt)
    ops.scatter(ops.LayerTable(dst), wl.page_ids, wl.slot_offsets, staging)
    oracle.scatter(dst_ref, wl.page_ids, wl.slot_offsets, ref, shape.layer_bytes)
    torch.cuda.synchronize()
    for l in range(shape.num_layers):
        assert np.array_equal(to_bits_np(dst[l], dt), dst_ref[l]), f"layer {l}"


@pytest.mark.parametrize("heads,dt", [(8, "bf16"), (16, "bf16"), (8, "e4m3"), (1, "bf16")])
@pytest.mark.parametrize("split", [0, 1, 2, 4, 8])
@pytest.mark.parametrize("n_pages", [1, 5, 64, 700])
def test_gather_split_units_match_oracle(gpu, tuning, heads, dt, split, n_pages):
    """The one-unit gather with each (page, layer) unit shared by several
    workgroups (launches of few units; split 0 = the launch policy's
    choice): the oracle's records, for pages of 32, 64, 16 and 4 KiB (the
    last cannot split) and one or all layers per launch."""
    print(f"case: gather split={split} H{heads} {dt} pages={n_pages}", flush=True)
    tuning("gather_split", split)
    shape = KVShape(3, heads, 128, 16, 1 if dt in FP8 else 2)
    nb = 2 * n_pages + 3
    rng = np.random.default_rng(n_pages + heads)
    ids = rng.permutation(nb)[:n_pages].astype(np.int32)
    offs = rng.permutation(n_pages).astype(np.int64) * shape.slot_bytes
    caches = rand_caches(shape, nb, dt, gpu, seed=21)
    table = ops.LayerTable(caches)
    host = [to_bits_np(c, dt) for c in caches]
    ref = np.zeros(n_pages * shape.slot_bytes, dtype=np.uint8)
    oracle.gather(host, ids, offs, ref, shape.layer_bytes)
    st = torch.zeros(ref.size, dtype=torch.uint8, device=gpu)
    ops.gather(table, ids, offs, st)
    torch.cuda.synchronize()
    assert np.array_equal(st.cpu().numpy(), ref)
    st.zero_()
    pg = ops.PreparedGather(table, ids, offs, st)
    for l in range(shape.num_layers):
        pg(l, 1, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert np.array_equal(st.cpu().numpy(), ref)


def test_device_tables_out_of_range_are_skipped_or_checked(gpu):
    """Device-resident tables are trusted: a page with an out-of-range block
    id or record offset is skipped (nothing written, no fault), the others
    are copied; ops.check_tables raises the host wrappers' errors for them."""
    print("case: device tables out of range", flush=True)
    shape = KVShape(2, 2, 64, 16, 2)
    nb = 8
    caches = rand_caches(shape, nb, "bf16", gpu, seed=14)
    st = torch.zeros(4 * shape.slot_bytes, dtype=torch.uint8, device=gpu)
    table = ops.LayerTable(caches)
    ids = torch.tensor([1, nb + 3, 4, -2], dtype=torch.int32, device=gpu)
    offs = torch.tensor([0, 1, 2, 3], dtype=torch.int64, device=gpu) * shape.slot_bytes
    ops.gather(table, ids, offs, st)
    torch.cuda.synchronize()
    rec = st.view(4, shape.num_layers, -1)
    for l in range(shape.num_layers):
        assert torch.equal(rec[0, l], caches[l][:, 1].reshape(-1).view(torch.uint8))
        assert torch.equal(rec[2, l], caches[l][:, 4].reshape(-1).view(torch.uint8))
    assert not rec[1].any() and not rec[3].any()
    with pytest.raises(IndexError, match="block id"):
        ops.check_tables(table, ids, offs, st, records_written=True)
    bad_offs = offs.clone()
    bad_offs[2] = 4 * shape.slot_bytes  # past the staging buffer
    with pytest.raises(IndexError, match="staging"):
        ops.check_tables(table, torch.tensor([1, 2, 4, 5], dtype=torch.int32, device=gpu),
                         bad_offs, st)
    ops.check_tables(table, torch.tensor([1, 2, 4, 5], dtype=torch.int32, device=gpu), offs, st,
                     records_written=True)


@pytest.mark.parametrize("shared", [True, False, None])
@pytest.mark.parametrize("heads", [8, 1])
def test_scatter_shared_records_hint_matches_oracle(gpu, heads, shared):
    """Pages reading the same records (one cached chunk placed in several
    requests) through dsr_scatter_ex with and without the shared-records
    hint, and with the hint inferred from host offsets: the oracle's bytes."""
    print(f"case: scatter shared={shared} H{heads}", flush=True)
    shape = KVShape(3, heads, 128, 16, 2)
    n_src, n = 6, 40
    rng = np.random.default_rng(heads)
    nb = 64
    src = rand_caches(shape, nb, "bf16", gpu, seed=12)
    st = torch.zeros(n_src * shape.slot_bytes, dtype=torch.uint8, device=gpu)
    ops.gather(ops.LayerTable(src), rng.permutation(nb)[:n_src].astype(np.int32),
               np.arange(n_src) * shape.slot_bytes, st)
    offs = rng.integers(0, n_src, n) * shape.slot_bytes
    ids = rng.permutation(nb)[:n].astype(np.int32)
    dst = rand_caches(shape, nb, "bf16", gpu, seed=13)
    ref = _np_layers(dst, "bf16")
    ops.scatter(ops.LayerTable(dst), ids, offs, st, shared_records=shared)
    oracle.scatter(ref, ids, offs, st.cpu().numpy(), shape.layer_bytes)
    torch.cuda.synchronize()
    for l in range(shape.num_layers):
        assert np.array_equal(to_bits_np(dst[l], "bf16"), ref[l]), f"layer {l}"


@pytest.mark.parametrize("dt", ["e4m3", "e5m2", "fp16"])
def test_gather_scatter_other_dtypes_bit_exact(gpu, dt):
    print(f"case: gather/scatter {dt}", flush=True)
    shape = KVShape(4, 8, 128, 16, 1 if dt in FP8 else 2)
    wl = workloads.ragged(shape, 5, 1, 300, seed=3, pool_slack=1.5)
    caches = rand_caches(shape, wl.num_blocks, dt, gpu, seed=4, scale=3.0)
    staging, ref = _gather_both(wl, caches, dt, gpu)
    torch.cuda.synchronize()
    assert np.array_equal(staging.cpu().numpy(), ref)
    dst = [torch.zeros_like(c) for c in caches]
    ops.scatter(ops.LayerTable(dst), wl.page_ids, wl.slot_offsets, staging)
    torch.cuda.synchronize()
    ids = torch.from_numpy(wl.page_ids.astype(np.int64)).to(gpu)
    for l in range(shape.num_layers):
        assert torch.equal(dst[l].view(torch.uint8)[:, ids], caches[l].view(torch.uint8)[:, ids])


def test_per_layer_launches_match_all_layer_launch(gpu):
    """save_kv_layer issues one launch per layer (layer0 = layer index)."""
    print("case: per-layer gather", flush=True)
    wl = workloads.config(1)
    caches = rand_caches(wl.shape, wl.num_blocks, "bf16", gpu, seed=5)
    table = ops.LayerTable(caches)
    full = torch.zeros(wl.staging_bytes, dtype=torch.uint8, device=gpu)
    ops.gather(table, wl.page_ids, wl.slot_offsets, full)
    per = torch.zeros_like(full)
    for l in range(wl.shape.num_layers):
        ops.gather(table, wl.page_ids, wl.slot_offsets, per, layers=(l, 1))
    torch.cuda.synchronize()
    assert torch.equal(full, per)


def test_prepared_gather_matches_gather(gpu):
    """ops.PreparedGather (tables bound once, one launch per layer on a given
    stream, as save_kv_layer uses it) writes what ops.gather writes, and
    rejects layer ranges outside the caches."""
    print("case: prepared gather", flush=True)
    wl = workloads.config(1)
    caches = rand_caches(wl.shape, wl.num_blocks, "bf16", gpu, seed=6)
    table = ops.LayerTable(caches)
    full = torch.zeros(wl.staging_bytes, dtype=torch.uint8, device=gpu)
    ops.gather(table, wl.page_ids, wl.slot_offsets, full)
    per = torch.zeros_like(full)
    side = torch.cuda.Stream(gpu)
    side.wait_stream(torch.cuda.current_stream(gpu))
    pg = ops.PreparedGather(table, torch.from_numpy(wl.page_ids).to(gpu),
                            torch.from_numpy(wl.slot_offsets).to(gpu), per)
    for l in reversed(range(wl.shape.num_layers)):
        pg(l, 1, side.cuda_stream)
    torch.cuda.current_stream(gpu).wait_stream(side)
    torch.cuda.synchronize()
    assert torch.equal(full, per)
    whole = torch.zeros_like(full)
    ops.PreparedGather(table, wl.page_ids, wl.slot_offsets, whole)(
        0, wl.shape.num_layers, torch.cuda.current_stream(gpu).cuda_stream)
    torch.cuda.synchronize()
    assert torch.equal(full, whole)
    for first, count in ((-1, 1), (wl.shape.num_layers, 1), (0, wl.shape.num_layers + 1)):
        with pytest.raises(IndexError):
            pg(first, count, side.cuda_stream)
    with pytest.raises(IndexError):  # tables checked once, at construction
        ops.PreparedGather(table, [wl.num_blocks], [0], per)


@pytest.mark.parametrize("heads,head_dim,dt", [
    (8, 128, "bf16"),   # 32 KiB pages: grouped kernel, one unit per workgroup
    (1, 128, "bf16"),   # 4 KiB: grouped, 8 units per workgroup
    (8, 128, "e4m3"),   # 16 KiB e4m3: contig kernel
    (1, 128, "e4m3"),   # 2 KiB e4m3: grouped
    (4, 96, "e4m3"),    # row-aligned kernel
])
def test_per_layer_rerotate_matches_all_layer_launch(gpu, heads, head_dim, dt):
    """Re-rotation launched per layer range (layers=(l, 1)) writes the same
    bytes as one launch over all layers: every kernel reads layer l's K scale
    at k_scale[layer0 + l]."""
    print(f"case: per-layer rerotate H{heads} D{head_dim} {dt}", flush=True)
    shape = KVShape(6, heads, head_dim, 16, 1 if dt in FP8 else 2)
    wl = workloads.ragged(shape, 4, 40, 400, seed=13, num_blocks=128)
    src = rand_caches(shape, wl.num_blocks, dt, gpu, seed=80, scale=40.0 if dt in FP8 else 1.0)
    st = torch.zeros(wl.staging_bytes, dtype=torch.uint8, device=gpu)
    ops.gather(ops.LayerTable(src), wl.page_ids, wl.slot_offsets, st)
    ridx = (np.arange(wl.n_pages) % 3 - 1).astype(np.int32)
    tabs = position.delta_tables([517, 32767], head_dim, 500000.0, device=gpu)
    ks = torch.linspace(0.05, 0.6, shape.num_layers, device=gpu) if dt in FP8 else None
    dst = np.random.default_rng(2).permutation(wl.num_blocks)[:wl.n_pages].astype(np.int32)
    one = [torch.zeros_like(c) for c in src]
    ops.scatter_rerotate(ops.LayerTable(one), dst, wl.slot_offsets, st, tabs, ridx, k_scale=ks)
    per = [torch.zeros_like(c) for c in src]
    t = ops.LayerTable(per)
    for l in range(shape.num_layers):
        ops.scatter_rerotate(t, dst, wl.slot_offsets, st, tabs, ridx, k_scale=ks,
                             layers=(l, 1))
    torch.cuda.synchronize()
    for l in range(shape.num_layers):
        assert torch.equal(one[l].view(torch.uint8), per[l].view(torch.uint8)), f"layer {l}"
    assert not torch.equal(one[0].view(torch.uint8), torch.zeros_like(one[0]).view(torch.uint8))


def test_strided_layout_block_major(gpu):
    """A cache allocated block-major (NB, 2, bs, H, D) and viewed as
    (2, NB, ...) has kv_stride = page, page_stride = 2 pages."""
    print("case: block-major layout", flush=True)
    shape = KVShape(3, 2, 64, 16, 2)
    nb = 40
    g = torch.Generator().manual_seed(6)
    caches = [torch.randn((nb, 2, 16, 2, 64), generator=g).to(torch.bfloat16).to(gpu)
              .permute(1, 0, 2, 3, 4) for _ in range(3)]
    wl = workloads.ragged(shape, 3, 1, 100, seed=7, num_blocks=nb)
    staging, ref = _gather_both(wl, [c.contiguous() for c in caches], "bf16", gpu)
    table = ops.LayerTable(caches)
    assert table.layout.kv_stride == table.layout.page_bytes
    st2 = torch.zeros_like(staging)
    ops.gather(table, wl.page_ids, wl.slot_offsets, st2)
    torch.cuda.synchronize()
    assert np.array_equal(st2.cpu().numpy(), ref)


def test_empty_and_single_page(gpu):
    print("case: empty/single", flush=True)
    shape = KVShape(2, 1, 64, 16, 2)
    caches = rand_caches(shape, 8, "bf16", gpu, seed=8)
    table = ops.LayerTable(caches)
    staging = torch.zeros(shape.slot_bytes, dtype=torch.uint8, device=gpu)
    ops.gather(table, np.zeros(0, np.int32), np.zeros(0, np.int64), staging)
    assert not staging.any()
    ops.gather(table, [7], [0], staging)  # last block of the pool
    torch.cuda.synchronize()
    exp = torch.cat([c[:, 7].reshape(-1).view(torch.uint8) for c in caches])
    assert torch.equal(staging, exp)


def test_out_of_range_rejected(gpu):
    shape = KVShape(2, 1, 64, 16, 2)
    caches = rand_caches(shape, 8, "bf16", gpu, seed=9)
    table = ops.LayerTable(caches)
    staging = torch.zeros(shape.slot_bytes, dtype=torch.uint8, device=gpu)
    with pytest.raises(IndexError):
        ops.gather(table, [8], [0], staging)
    with pytest.raises(IndexError):
        ops.gather(table, [0], [16], staging)
    with pytest.raises(ValueError):
        ops.gather(table, [0], [8], torch.zeros(2 * shape.slot_bytes, dtype=torch.uint8, device=gpu))


def test_device_tables_out_of_range_skipped(gpu):
    """Device-side tables are not validated on the host; the kernel skips
    entries outside the pool or the staging buffer instead of faulting."""
    print("case: device tables skip", flush=True)
    shape = KVShape(2, 1, 64, 16, 2)
    caches = rand_caches(shape, 8, "bf16", gpu, seed=10)
    table = ops.LayerTable(caches)
    staging = torch.zeros(2 * shape.slot_bytes, dtype=torch.uint8, device=gpu)
    ids = torch.tensor([3, 1000, -1, 2], dtype=torch.int32, device=gpu)
    offs = torch.tensor([0, 0, 0, 1 << 40], dtype=torch.int64, device=gpu)
    ops.gather(table, ids, offs, staging)
    torch.cuda.synchronize()
    exp = torch.cat([c[:, 3].reshape(-1).view(torch.uint8) for c in caches])
    assert torch.equal(staging[: shape.slot_bytes], exp)
    assert not staging[shape.slot_bytes:].any()


# ---------------------------------------------------------------------------
# fused re-rotation


def _rerotate_case(gpu, dt, style, head_dim, rot_dim, heads=4, layers=3, seed=0,
                   deltas=(0, 1, 517, 32767, 123), theta=500000.0, scale=1.0,
                   inputs=None):
    shape = KVShape(layers, heads, head_dim, 16, 1 if dt in FP8 else 2)
    rng = np.random.default_rng(seed)
    chunk_pages = [int(x) for x in rng.integers(1, 4, size=len(deltas))]
    n = sum(chunk_pages)
    nb = n + 5
    src_caches = rand_caches(shape, nb, dt, gpu, seed=seed + 1, scale=scale)
    # records: gather every block of a source pool into staging
    staging = torch.zeros(n * shape.slot_bytes, dtype=torch.uint8, device=gpu)
    offs = np.arange(n, dtype=np.int64) * shape.slot_bytes
    ops.gather(ops.LayerTable(src_caches), rng.permutation(nb)[:n].astype(np.int32), offs, staging)
    dst = rand_caches(shape, nb, dt, gpu, seed=seed + 2)
    dst_ref = [to_bits_np(c, dt) for c in dst]
    page_ids = rng.permutation(nb)[:n].astype(np.int32)
    ridx, uniq = position.page_rope_index(chunk_pages, deltas)
    tabs = position.delta_tables(uniq or [0], rot_dim, theta, device=gpu)
    k_scale = None
    ks_np = None
    if dt in FP8:
        ks_np = (rng.random(layers).astype(np.float32) * 0.5 + 0.01)
        k_scale = torch.from_numpy(ks_np).to(gpu)
    ops.scatter_rerotate(ops.LayerTable(dst), page_ids, offs, staging, tabs, ridx,
                         rot_dim=rot_dim, style=style, k_scale=k_scale)
    page_delta = np.repeat(np.asarray(deltas, np.int64), chunk_pages)
    oracle.scatter_rerotate(
        dst_ref, page_ids, offs, staging.cpu().numpy(), shape.layer_bytes,
        dtype=ORC_DT[dt], rot_dim=rot_dim, style=0 if style == "neox" else 1,
        stored_pos=np.zeros(n, np.int64), new_pos=page_delta, rotate=page_delta != 0,
        theta=theta, k_scale=ks_np)
    torch.cuda.synchronize()
    if inputs is not None:  # the records and offsets, for float64 checks
        inputs.update(staging=staging.cpu().numpy(), offsets=offs)
    return shape, dst, dst_ref, page_ids, page_delta


def _exact_rotation(staging, offsets, shape, layer, page_delta, rot_dim, style, theta):
    """Float64 rotation of each page's stored bf16 K by its delta (no
    rounding): (n_pages, bs, H, D) values. Pairs (j, j + R/2) for neox,
    (2j, 2j + 1) for gptj; dims past rot_dim unchanged."""
    n = len(offsets)
    k = np.stack([staging[o + layer * shape.layer_bytes:
                          o + layer * shape.layer_bytes + shape.page_bytes]
                  for o in offsets]).view(np.uint16)
    x = (k.astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    x = x.reshape(n, shape.block_size, shape.num_heads, shape.head_dim)
    half = rot_dim // 2
    inv = np.power(float(theta), -2.0 * np.arange(half) / rot_dim)
    ang = np.asarray(page_delta, np.float64)[:, None] * inv[None, :]
    c = np.cos(ang)[:, None, None, :]
    s_ = np.sin(ang)[:, None, None, :]
    y = x.copy()
    if style == "neox":
        a, b = x[..., :half], x[..., half:rot_dim]
        y[..., :half] = a * c - b * s_
        y[..., half:rot_dim] = b * c + a * s_
    else:
        a, b = x[..., 0:rot_dim:2], x[..., 1:rot_dim:2]
        y[..., 0:rot_dim:2] = a * c - b * s_
        y[..., 1:rot_dim:2] = b * c + a * s_
    return y


@pytest.mark.parametrize(
    "dt,style,head_dim,rot_dim",
    [
        ("bf16", "neox", 128, 128),
        ("bf16", "gptj", 128, 128),
        ("bf16", "neox", 128, 64),
        ("bf16", "neox", 64, 64),
        ("fp16", "neox", 128, 128),
        ("fp16", "gptj", 256, 128),
        ("e4m3", "neox", 128, 128),
        ("e4m3", "gptj", 128, 96),
        ("e5m2", "neox", 128, 128),
        ("e5m2", "gptj", 128, 96),
        ("e5m2", "neox", 192, 192),
        ("e5m2", "neox", 128, 40),
        # partner distance not a power of two: the row-aligned kernel
        ("bf16", "neox", 80, 80),
        ("fp16", "neox", 96, 96),
        ("e4m3", "neox", 192, 192),
        # rotary widths that are not whole vectors: the LDS kernel
        ("bf16", "neox", 96, 24),
        ("bf16", "neox", 80, 20),
        ("fp16", "gptj", 80, 20),
        ("e4m3", "neox", 128, 40),
        ("e4m3", "gptj", 64, 24),
        ("bf16", "neox", 256, 254),
    ],
)
def test_rerotate_matches_oracle(gpu, dt, style, head_dim, rot_dim):
    print(f"case: rerotate {dt} {style} D{head_dim} R{rot_dim}", flush=True)
    inputs = {}
    shape, dst, dst_ref, page_ids, page_delta = _rerotate_case(
        gpu, dt, style, head_dim, rot_dim, scale=40.0 if dt in FP8 else 1.0, inputs=inputs)
    for l in range(shape.num_layers):
        got = to_bits_np(dst[l], dt)
        ref = dst_ref[l]
        # V (index 1) and untouched blocks: bit-exact
        assert np.array_equal(got[1], ref[1])
        ok, msg = rotation_within_tolerance(got[0], ref[0], dt)
        assert ok, f"layer {l}: {msg}"
        # un-rotated pages (delta 0) are bit-exact copies
        zero_pages = page_ids[page_delta == 0]
        assert np.array_equal(got[0][zero_pages], ref[0][zero_pages])
        if dt == "bf16":
            # atol 1e-2 (unscaled) against the unrounded float64 rotation of
            # the stored K, for |value| < 4: there half a bf16 ulp is at most
            # 2^-8, so a correctly rounded result is within 1e-2. From 4 up a
            # bf16 ulp is 2^-5 > 2e-2 and the 1-ulp check above is the bar.
            exact = _exact_rotation(inputs["staging"], inputs["offsets"], shape, l,
                                    page_delta, rot_dim, style, 500000.0)
            a = (got[0][page_ids].astype(np.uint32) << 16).view(np.float32).astype(np.float64)
            small = np.abs(exact) < 4.0
            assert small.mean() > 0.99
            err = np.abs(a - exact)[small]
            assert err.max() <= 1e-2, f"layer {l}: max abs err {err.max():.3g} > 1e-2"


@pytest.mark.parametrize("dt,head_dim", [("bf16", 80), ("fp16", 96), ("e4m3", 192)])
def test_rerotate_pair_task_kernel_matches_oracle(gpu, tuning, dt, head_dim):
    """The pair-task kernel (kept for rows of more than 64 vectors), forced
    on the shapes the row-aligned kernel serves by default."""
    print(f"case: rerotate pair-task {dt} D{head_dim}", flush=True)
    tuning("rot_kernel", "pairs")
    shape, dst, dst_ref, page_ids, page_delta = _rerotate_case(
        gpu, dt, "neox", head_dim, head_dim, scale=40.0 if dt in FP8 else 1.0)
    for l in range(shape.num_layers):
        got = to_bits_np(dst[l], dt)
        assert np.array_equal(got[1], dst_ref[l][1])
        ok, msg = rotation_within_tolerance(got[0], dst_ref[l][0], dt)
        assert ok, f"layer {l}: {msg}"


@pytest.mark.parametrize("dt", ["bf16", "e4m3"])
def test_rerotate_single_kv_head(gpu, dt):
    """One KV head per page (a TP8 rank of a 70B model: 4 KiB bf16 pages,
    2 KiB e4m3): rows of 256 / 128 bytes."""
    print(f"case: rerotate single head {dt}", flush=True)
    shape, dst, dst_ref, page_ids, page_delta = _rerotate_case(
        gpu, dt, "neox", 128, 128, heads=1, layers=5, seed=9,
        scale=40.0 if dt in FP8 else 1.0)
    for l in range(shape.num_layers):
        got = to_bits_np(dst[l], dt)
        assert np.array_equal(got[1], dst_ref[l][1])
        ok, msg = rotation_within_tolerance(got[0], dst_ref[l][0], dt)
        assert ok, f"layer {l}: {msg}"


def test_rerotate_inverse_is_identity(gpu):
    """Rotating by +d then -d returns the input within 2 bf16 ulps."""
    print("case: rerotate inverse", flush=True)
    shape = KVShape(2, 8, 128, 16, 2)
    nb = 12
    caches = rand_caches(shape, nb, "bf16", gpu, seed=21)
    ids = np.arange(nb, dtype=np.int32)
    offs = np.arange(nb, dtype=np.int64) * shape.slot_bytes
    st = torch.zeros(nb * shape.slot_bytes, dtype=torch.uint8, device=gpu)
    ops.gather(ops.LayerTable(caches), ids, offs, st)
    tabs = position.delta_tables([12345, -12345], 128, 500000.0, device=gpu)
    mid = [torch.zeros_like(c) for c in caches]
    ops.scatter_rerotate(ops.LayerTable(mid), ids, offs, st, tabs, np.zeros(nb, np.int32))
    st2 = torch.zeros_like(st)
    ops.gather(ops.LayerTable(mid), ids, offs, st2)
    back = [torch.zeros_like(c) for c in caches]
    ops.scatter_rerotate(ops.LayerTable(back), ids, offs, st2, tabs, np.ones(nb, np.int32))
    torch.cuda.synchronize()
    for c, b in zip(caches, back):
        ok, msg = rotation_within_tolerance(to_bits_np(b, "bf16"), to_bits_np(c, "bf16"),
                                            "bf16", rel_row=2.0 ** -7)
        assert ok, msg
        assert torch.equal(b[1], c[1])


def test_rerotate_bad_geometry_rejected(gpu):
    shape = KVShape(1, 1, 64, 16, 1)
    caches = rand_caches(shape, 2, "e4m3", gpu, seed=22)
    st = torch.zeros(shape.slot_bytes, dtype=torch.uint8, device=gpu)
    tabs = position.delta_tables([5], 66, device=gpu)
    with pytest.raises(DaserKVError):
        # a rotary width beyond head_dim
        ops.scatter_rerotate(ops.LayerTable(caches), [0], [0], st, tabs, [0], rot_dim=66,
                             k_scale=torch.ones(1, device=gpu))


@pytest.mark.parametrize("dt", ["bf16", "e4m3", "e5m2"])
def test_rerotate_special_values(gpu, dt):
    """NaN, +-Inf (bf16, e5m2), +-0, subnormals and the 8-bit extremes follow
    the oracle: NaN stays canonical NaN, zero delta is bit-exact (infinities
    included), the 8-bit formats saturate."""
    print(f"case: rerotate special values {dt}", flush=True)
    shape = KVShape(2, 2, 64, 16, 1 if dt in FP8 else 2)
    nb = 4
    caches = rand_caches(shape, nb, dt, gpu, seed=40, scale=30.0 if dt in FP8 else 1.0)
    if dt == "bf16":
        special = torch.tensor([float("nan"), float("inf"), -float("inf"), 0.0, -0.0,
                                1e-40, -3e-39, 65504.0], dtype=torch.float32).to(torch.bfloat16)
        bits = special.view(torch.int16)
        for c in caches:
            v = c.view(torch.int16)
            v[0, :, 0, 0, :8] = bits.to(gpu)          # first-half elements
            v[0, :, 1, 1, 32:40] = bits.to(gpu)       # their neox partners
    else:
        codes = torch.tensor([0x7F, 0xFF, 0x00, 0x80, 0x01, 0x81, 0x7E, 0xFE] if dt == "e4m3"
                             else [0x7F, 0xFD, 0x00, 0x80, 0x01, 0x7C, 0xFC, 0x7B],
                             dtype=torch.uint8)
        for c in caches:
            v = c.view(torch.uint8)
            v[0, :, 0, 0, :8] = codes.to(gpu)
            v[0, :, 2, 1, 32:40] = codes.to(gpu)
    ids = np.arange(nb, dtype=np.int32)
    offs = ids.astype(np.int64) * shape.slot_bytes
    st = torch.zeros(nb * shape.slot_bytes, dtype=torch.uint8, device=gpu)
    ops.gather(ops.LayerTable(caches), ids, offs, st)
    dst = [torch.zeros_like(c) for c in caches]
    deltas = [0, 1, 777, 32767]
    ridx, uniq = position.page_rope_index([1] * nb, deltas)
    tabs = position.delta_tables(uniq, 64, 500000.0, device=gpu)
    ks = torch.tensor([0.5, 2.0], device=gpu) if dt in FP8 else None
    ops.scatter_rerotate(ops.LayerTable(dst), ids, offs, st, tabs, ridx, k_scale=ks)
    ref = [np.zeros_like(to_bits_np(c, dt)) for c in caches]
    oracle.scatter_rerotate(ref, ids, offs, st.cpu().numpy(), shape.layer_bytes,
                            dtype=ORC_DT[dt], rot_dim=64, style=0,
                            stored_pos=np.zeros(nb, np.int64), new_pos=np.asarray(deltas),
                            rotate=np.asarray(deltas) != 0, theta=500000.0,
                            k_scale=None if ks is None else np.float32([0.5, 2.0]))
    torch.cuda.synchronize()
    for l in range(2):
        got = to_bits_np(dst[l], dt)
        assert np.array_equal(got[1], ref[l][1])
        assert np.array_equal(got[0][0], ref[l][0][0])  # zero delta: bit-exact
        nan_ref = np.isnan(oracle.decode(ORC_DT[dt], ref[l][0]))
        nan_got = np.isnan(oracle.decode(ORC_DT[dt], got[0]))
        assert np.array_equal(nan_ref, nan_got)
        assert np.array_equal(got[0][nan_got], ref[l][0][nan_ref])  # canonical NaN bits
        ok, msg = oracle.rotation_within_tolerance(np.where(nan_got, 0, got[0]),
                                                   np.where(nan_ref, 0, ref[l][0]), ORC_DT[dt])
        assert ok, msg


@pytest.mark.parametrize("shape", [
    None,                          # config 1, Qwen2-0.5B: 256-byte rows (16 vectors)
    KVShape(6, 1, 64, 16, 2),      # 128-byte rows
    KVShape(5, 2, 128, 16, 2),     # 512-byte rows (32 vectors)
    KVShape(4, 4, 128, 16, 2),     # 1 KiB rows: the large-row kernel
    KVShape(5, 1, 128, 16, 1),     # e4m3, 128-byte rows
    KVShape(3, 1, 32, 32, 2),      # 64-byte rows (4 vectors), block size 32
    KVShape(3, 1, 16, 8, 1),       # 16-byte rows (1 vector)
    KVShape(3, 1, 64, 12, 2),      # 128-byte rows, block size 12 (not a power of two)
], ids=["cfg1", "row128", "row512", "row1k", "e4m3_row128", "row64_bs32", "row16",
        "row128_bs12"])
@pytest.mark.parametrize("unroll,form", [("default", "host"), ("4", "host"),
                                          ("default", "device")])
def test_slots_gather_scatter_match_oracle(gpu, tuning, shape, unroll, form):
    """slot_mapping-driven token gather/scatter with ragged requests, partial
    last pages and padding tokens, at each row-size class of the kernels
    (rows of <= 8 vectors: the packed kernel, at both unrolls). Host tables
    scatter whole pages through the page kernel and the rest through the
    token kernel; device tables take the token kernel for every token."""
    print(f"case: slots gather/scatter {shape} unroll {unroll} {form}", flush=True)
    if unroll != "default":
        tuning("slots_unroll", int(unroll))
    wl = workloads.config(1) if shape is None else workloads.ragged(
        shape, 8, 100, 2000, seed=3, num_blocks=1024)
    shape = wl.shape
    dt = "e4m3" if shape.elem_bytes == 1 else "bf16"
    caches = rand_caches(shape, wl.num_blocks, dt, gpu, seed=50)
    tables, k = [], 0
    for n in wl.req_pages:
        tables.append(wl.page_ids[k:k + n].tolist())
        k += n
    row = shape.num_heads * shape.head_dim * shape.elem_bytes
    sm = ops.slot_mapping_for(tables, wl.req_tokens, shape.block_size)
    ro = ops.token_row_offsets(wl.req_tokens, shape.slot_bytes, shape.block_size, row)
    pad = np.arange(0, sm.size, 97)
    sm[pad] = -1
    st = torch.zeros(wl.staging_bytes, dtype=torch.uint8, device=gpu)
    ops.gather_slots(ops.LayerTable(caches), sm, ro, st)
    ref = np.zeros(wl.staging_bytes, dtype=np.uint8)
    host = [to_bits_np(c, dt) for c in caches]
    oracle.gather_slots(host, sm, ro, ref, shape.layer_bytes)
    torch.cuda.synchronize()
    assert np.array_equal(st.cpu().numpy(), ref)
    dst = [torch.zeros_like(c) for c in caches]
    if form == "device":
        ops.scatter_slots(ops.LayerTable(dst), torch.from_numpy(sm).to(gpu),
                          torch.from_numpy(ro).to(gpu), st)
    else:
        ops.scatter_slots(ops.LayerTable(dst), sm, ro, st)
    dref = [np.zeros_like(h) for h in host]
    oracle.scatter_slots(dref, sm, ro, ref, shape.layer_bytes)
    torch.cuda.synchronize()
    for d, r in zip(dst, dref):
        assert np.array_equal(to_bits_np(d, dt), r)


def test_slots_duplicates_keep_the_last_token(gpu):
    """Host tables in which two tokens target the same cache slot (scatter)
    or the same record row (gather): the last token's bytes land, as the
    oracle's sequential loop leaves them; the caller's table is not
    modified."""
    print("case: slots duplicates keep the last token", flush=True)
    shape = KVShape(3, 2, 64, 16, 2)
    nb = 16
    caches = rand_caches(shape, nb, "bf16", gpu, seed=61)
    row = shape.num_heads * shape.head_dim * shape.elem_bytes
    host = [to_bits_np(c, "bf16") for c in caches]
    # scatter: tokens 1 and 4 both target slot 37, tokens 2 and 5 slot 40
    sm = np.array([5, 37, 40, 70, 37, 40, -1, 90], np.int64)
    ro = np.arange(sm.size, dtype=np.int64) * row
    sm_before = sm.copy()
    rng = np.random.default_rng(62)
    rec = rng.integers(0, 256, size=shape.slot_bytes, dtype=np.uint8)
    st = torch.from_numpy(rec).to(gpu)
    ops.scatter_slots(ops.LayerTable(caches), sm, ro, st)
    oracle.scatter_slots(host, sm, ro, rec, shape.layer_bytes)
    torch.cuda.synchronize()
    assert np.array_equal(sm, sm_before)
    for c, r in zip(caches, host):
        assert np.array_equal(to_bits_np(c, "bf16"), r)
    # gather: tokens 0 and 3 write record row 2, tokens 1 and 6 row 5
    ro2 = np.array([2, 5, 0, 2, 1, 3, 5], np.int64) * row
    sm2 = np.array([3, 17, 33, 49, 65, 81, 97], np.int64)
    st2 = torch.zeros(shape.slot_bytes, dtype=torch.uint8, device=gpu)
    ops.gather_slots(ops.LayerTable(caches), sm2, ro2, st2)
    ref = np.zeros(shape.slot_bytes, dtype=np.uint8)
    oracle.gather_slots(host, sm2, ro2, ref, shape.layer_bytes)
    torch.cuda.synchronize()
    assert np.array_equal(st2.cpu().numpy(), ref)


def test_slots_gather_equals_page_gather_for_full_pages(gpu):
    print("case: slots == pages", flush=True)
    shape = KVShape(4, 8, 128, 16, 2)
    wl = workloads.ragged(shape, 6, 1, 40, seed=51, pool_slack=1.3)
    toks = [n * 16 for n in wl.req_pages]  # whole pages
    caches = rand_caches(shape, wl.num_blocks, "bf16", gpu, seed=52)
    table = ops.LayerTable(caches)
    tables, k = [], 0
    for n in wl.req_pages:
        tables.append(wl.page_ids[k:k + n].tolist())
        k += n
    a = torch.zeros(wl.staging_bytes, dtype=torch.uint8, device=gpu)
    b = torch.zeros_like(a)
    ops.gather(table, wl.page_ids, wl.slot_offsets, a)
    ops.gather_slots(table, ops.slot_mapping_for(tables, toks, 16),
                     ops.token_row_offsets(toks, shape.slot_bytes, 16, 8 * 128 * 2), b)
    torch.cuda.synchronize()
    assert torch.equal(a, b)


def test_large_page_geometry(gpu):
    """512 KiB pages (block_size 32, 32 heads, head_dim 256): multi-round
    copies and a 32-lane neox partner distance."""
    print("case: large pages", flush=True)
    shape = KVShape(2, 32, 256, 32, 2)
    wl = workloads.ragged(shape, 3, 1, 100, seed=70, pool_slack=1.5)
    caches = rand_caches(shape, wl.num_blocks, "bf16", gpu, seed=71)
    staging, ref = _gather_both(wl, caches, "bf16", gpu)
    torch.cuda.synchronize()
    assert np.array_equal(staging.cpu().numpy(), ref)
    dst = [torch.zeros_like(c) for c in caches]
    ridx = np.zeros(wl.n_pages, np.int32)
    tabs = position.delta_tables([999], 256, 500000.0, device=gpu)
    ops.scatter_rerotate(ops.LayerTable(dst), wl.page_ids, wl.slot_offsets, staging, tabs, ridx)
    dref = [np.zeros_like(to_bits_np(c, "bf16")) for c in caches]
    oracle.scatter_rerotate(dref, wl.page_ids, wl.slot_offsets, ref, shape.layer_bytes,
                            dtype=oracle.BF16, rot_dim=256, style=oracle.NEOX,
                            stored_pos=np.zeros(wl.n_pages, np.int64),
                            new_pos=np.full(wl.n_pages, 999), rotate=np.ones(wl.n_pages),
                            theta=500000.0)
    torch.cuda.synchronize()
    for d, r in zip(dst, dref):
        got = to_bits_np(d, "bf16")
        assert np.array_equal(got[1], r[1])
        ok, msg = oracle.rotation_within_tolerance(got[0], r[0], oracle.BF16)
        assert ok, msg


# ---------------------------------------------------------------------------
# pages of whole 4 KiB slices: several units per workgroup


@pytest.mark.parametrize("layers,heads,head_dim,dt", [
    (7, 1, 128, "bf16"),   # 4 KiB pages: one slice per unit
    (5, 2, 128, "bf16"),   # 8 KiB: two slices per unit
    (6, 2, 64, "bf16"),    # Qwen2-0.5B geometry
    (5, 2, 128, "e4m3"),   # 4 KiB e4m3
    (5, 1, 128, "e4m3"),   # 2 KiB: two units per workgroup slice
    (4, 1, 64, "bf16"),    # 2 KiB
    (3, 1, 64, "e4m3"),    # 1 KiB: one unit per wave
])
@pytest.mark.parametrize("group_cap", ["1", "2", "3", ""])
def test_grouped_units_match_oracle(gpu, tuning, layers, heads, head_dim, dt, group_cap):
    """Groups span layer boundaries (3 pages, fewer than a group) and end
    part-way; every grouping (1 = the one-unit kernels) gives the oracle's
    bytes for gather, scatter and re-rotation."""
    print(f"case: grouped L{layers} H{heads} D{head_dim} {dt} cap={group_cap!r}", flush=True)
    if group_cap:
        tuning("units_per_group", int(group_cap))
    else:
        tuning("units_per_group", 0)
    shape = KVShape(layers, heads, head_dim, 16, 1 if dt in FP8 else 2)
    nb = 9
    src = rand_caches(shape, nb, dt, gpu, seed=60, scale=40.0 if dt in FP8 else 1.0)
    ids = np.array([5, 0, 7], dtype=np.int32)
    offs = np.array([2, 0, 1], dtype=np.int64) * shape.slot_bytes
    staging = torch.zeros(3 * shape.slot_bytes, dtype=torch.uint8, device=gpu)
    ops.gather(ops.LayerTable(src), ids, offs, staging)
    ref = np.zeros(3 * shape.slot_bytes, dtype=np.uint8)
    src_np = _np_layers(src, dt)
    oracle.gather(src_np, ids, offs, ref, shape.layer_bytes)
    torch.cuda.synchronize()
    assert np.array_equal(staging.cpu().numpy(), ref)

    dst_ids = np.array([4, 8, 1], dtype=np.int32)
    dst = [torch.zeros_like(c) for c in src]
    ops.scatter(ops.LayerTable(dst), dst_ids, offs, staging)
    dref = [np.zeros_like(a) for a in src_np]
    oracle.scatter(dref, dst_ids, offs, ref, shape.layer_bytes)
    torch.cuda.synchronize()
    for l in range(layers):
        assert np.array_equal(to_bits_np(dst[l], dt), dref[l])

    deltas = [0, 517, 32767]
    ridx, uniq = position.page_rope_index([1, 1, 1], deltas)
    tabs = position.delta_tables(uniq, head_dim, 500000.0, device=gpu)
    ks_np = None
    k_scale = None
    if dt in FP8:
        ks_np = np.linspace(0.05, 0.5, layers).astype(np.float32)
        k_scale = torch.from_numpy(ks_np).to(gpu)
    rot = [torch.zeros_like(c) for c in src]
    ops.scatter_rerotate(ops.LayerTable(rot), dst_ids, offs, staging, tabs, ridx,
                         k_scale=k_scale)
    rref = [np.zeros_like(a) for a in src_np]
    d = np.asarray(deltas, np.int64)
    oracle.scatter_rerotate(rref, dst_ids, offs, ref, shape.layer_bytes, dtype=ORC_DT[dt],
                            rot_dim=head_dim, style=0, stored_pos=np.zeros(3, np.int64),
                            new_pos=d, rotate=d != 0, theta=500000.0, k_scale=ks_np)
    torch.cuda.synchronize()
    for l in range(layers):
        got = to_bits_np(rot[l], dt)
        assert np.array_equal(got[1], rref[l][1])
        assert np.array_equal(got[0][4], rref[l][0][4])  # delta 0: copy
        ok, msg = rotation_within_tolerance(got[0], rref[l][0], dt)
        assert ok, f"layer {l}: {msg}"


@pytest.mark.parametrize("group_cap", ["1", ""])
def test_grouped_units_skip_out_of_range(gpu, tuning, group_cap):
    """Device tables with an out-of-range block inside a group: that unit is
    skipped in every layer, its neighbours in the group still move."""
    print(f"case: grouped skip cap={group_cap!r}", flush=True)
    if group_cap:
        tuning("units_per_group", int(group_cap))
    else:
        tuning("units_per_group", 0)
    shape = KVShape(5, 1, 128, 16, 2)
    src = rand_caches(shape, 8, "bf16", gpu, seed=61)
    staging = torch.zeros(3 * shape.slot_bytes, dtype=torch.uint8, device=gpu)
    ids = torch.tensor([3, 1000, 6], dtype=torch.int32, device=gpu)
    offs = torch.tensor([0, 1, 2], dtype=torch.int64, device=gpu) * shape.slot_bytes
    ops.gather(ops.LayerTable(src), ids, offs, staging)
    torch.cuda.synchronize()
    for i, b in ((0, 3), (2, 6)):
        exp = torch.cat([c[:, b].reshape(-1).view(torch.uint8) for c in src])
        assert torch.equal(staging[i * shape.slot_bytes:(i + 1) * shape.slot_bytes], exp)
    assert not staging[shape.slot_bytes:2 * shape.slot_bytes].any()
    dst = [torch.zeros_like(c) for c in src]
    dids = torch.tensor([1, -1, 4], dtype=torch.int32, device=gpu)
    ops.scatter(ops.LayerTable(dst), dids, offs, staging)
    tabs = position.delta_tables([300], 128, 500000.0, device=gpu)
    rot = [torch.zeros_like(c) for c in src]
    ridx = torch.tensor([0, 0, -1], dtype=torch.int32, device=gpu)
    ops.scatter_rerotate(ops.LayerTable(rot), dids, offs, staging, tabs, ridx)
    torch.cuda.synchronize()
    for l in range(shape.num_layers):
        assert torch.equal(dst[l][:, 1], src[l][:, 3])
        assert torch.equal(dst[l][:, 4], src[l][:, 6])
        assert torch.equal(rot[l][:, 4], src[l][:, 6])       # no table: copy
        assert torch.equal(rot[l][1, 1], src[l][1, 3])       # V copied
        assert not torch.equal(rot[l][0, 1], src[l][0, 3])   # K rotated
        others = [b for b in range(8) if b not in (1, 4)]
        assert not dst[l][:, others].view(torch.int16).any()
        assert not rot[l][:, others].view(torch.int16).any()


@pytest.mark.parametrize("layers,heads,head_dim,dt", [
    (4, 8, 128, "bf16"),    # one-unit kernels
    (7, 1, 128, "bf16"),    # grouped (4 KiB pages)
    (5, 1, 128, "e4m3"),    # grouped (2 KiB pages)
])
def test_launch_split_matches_single_launch(gpu, tuning, layers, heads, head_dim, dt):
    """Calls whose workgroups exceed one launch's limit run as several
    launches over page (token) ranges; forced here with a limit of 16
    workgroups, every entry point writes the same bytes as one launch."""
    print(f"case: launch split L{layers} H{heads} {dt}", flush=True)
    shape = KVShape(layers, heads, head_dim, 16, 1 if dt in FP8 else 2)
    wl = workloads.ragged(shape, 6, 40, 700, seed=12, num_blocks=256)
    src = rand_caches(shape, wl.num_blocks, dt, gpu, seed=70, scale=40.0 if dt in FP8 else 1.0)
    ridx = np.arange(wl.n_pages, dtype=np.int32) % 3 - 1  # -1 (copy), 0, 1
    tabs = position.delta_tables([517, 32767], head_dim, 500000.0, device=gpu)
    ks = torch.linspace(0.05, 0.5, layers, device=gpu) if dt in FP8 else None
    tables, k = [], 0
    for n in wl.req_pages:
        tables.append(wl.page_ids[k:k + n].tolist())
        k += n
    row = heads * head_dim * shape.elem_bytes
    sm = ops.slot_mapping_for(tables, wl.req_tokens, 16)
    ro = ops.token_row_offsets(wl.req_tokens, shape.slot_bytes, 16, row)

    def run():
        table = ops.LayerTable(src)
        st = torch.zeros(wl.staging_bytes, dtype=torch.uint8, device=gpu)
        ops.gather(table, wl.page_ids, wl.slot_offsets, st)
        st2 = torch.zeros_like(st)
        ops.gather_slots(table, sm, ro, st2)
        outs = [st, st2]
        perm = np.random.default_rng(1).permutation(wl.num_blocks)[:wl.n_pages].astype(np.int32)
        for kind in ("scatter", "rerotate", "slots"):
            dst = [torch.zeros_like(c) for c in src]
            t = ops.LayerTable(dst)
            if kind == "scatter":
                ops.scatter(t, perm, wl.slot_offsets, st)
            elif kind == "rerotate":
                ops.scatter_rerotate(t, perm, wl.slot_offsets, st, tabs, ridx, k_scale=ks)
            else:
                ops.scatter_slots(t, sm, ro, st2)
            outs += [d.view(torch.uint8).clone() for d in dst]
        torch.cuda.synchronize()
        return outs

    tuning("max_wg_per_launch", 0)
    one = run()
    tuning("max_wg_per_launch", 16)
    split = run()
    for i, (a, b) in enumerate(zip(one, split)):
        assert torch.equal(a, b), f"output {i}"
    assert one[0].any() and one[2].any()


def test_hip_graph_capture_and_replay(gpu):
    """With device-resident tables the entry points allocate, synchronise and
    memset nothing, so a step's gather / scatter / re-rotation can be
    captured into a HIP graph. Each of three replays, with other work and
    new inputs in between, equals the eager result."""
    print("case: graph capture", flush=True)
    shape = KVShape(4, 2, 128, 16, 2)  # 8 KiB pages
    wl = workloads.ragged(shape, 4, 40, 400, seed=14, num_blocks=128)
    src = rand_caches(shape, wl.num_blocks, "bf16", gpu, seed=90)
    table_s = ops.LayerTable(src)
    ids = torch.from_numpy(wl.page_ids.astype(np.int32)).to(gpu)
    offs = torch.from_numpy(wl.slot_offsets).to(gpu)
    dst_ids = torch.from_numpy(np.random.default_rng(3).permutation(wl.num_blocks)[:wl.n_pages]
                               .astype(np.int32)).to(gpu)
    ridx = torch.from_numpy((np.arange(wl.n_pages) % 2).astype(np.int32) - 1).to(gpu)
    tabs = position.delta_tables([4096], 128, 500000.0, device=gpu)
    st = torch.zeros(wl.staging_bytes, dtype=torch.uint8, device=gpu)
    dst = [torch.zeros_like(c) for c in src]
    rot = [torch.zeros_like(c) for c in src]
    tok = [torch.zeros_like(c) for c in src]
    table_d, table_r, table_t = ops.LayerTable(dst), ops.LayerTable(rot), ops.LayerTable(tok)
    # the token forms: the same requests by slot_mapping, each request's
    # tokens re-rotated by its own table or (odd requests) copied
    tables, k = [], 0
    for n in wl.req_pages:
        tables.append(wl.page_ids[k:k + n].tolist())
        k += n
    row = shape.num_heads * shape.head_dim * shape.elem_bytes
    sm = torch.from_numpy(ops.slot_mapping_for(tables, wl.req_tokens, shape.block_size)).to(gpu)
    ro = torch.from_numpy(ops.token_row_offsets(wl.req_tokens, shape.slot_bytes,
                                                shape.block_size, row)).to(gpu)
    tidx = torch.from_numpy(np.repeat((np.arange(len(wl.req_tokens)) % 2).astype(np.int32) - 1,
                                      wl.req_tokens)).to(gpu)
    st_t = torch.zeros_like(st)

    def step():
        ops.gather(table_s, ids, offs, st)
        ops.scatter(table_d, dst_ids, offs, st)
        ops.scatter_rerotate(table_r, dst_ids, offs, st, tabs, ridx)
        ops.gather_slots(table_s, sm, ro, st_t)
        ops.scatter_slots_rerotate(table_t, sm, ro, st_t, tabs, tidx)

    def snapshot():
        torch.cuda.synchronize()
        return [st.clone(), st_t.clone()] + [t.clone() for t in dst + rot + tok]

    side = torch.cuda.Stream(gpu)
    side.wait_stream(torch.cuda.current_stream(gpu))
    with torch.cuda.stream(side):
        step()  # warm-up on the capture stream
    torch.cuda.current_stream(gpu).wait_stream(side)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        step()
    for rep in range(3):
        for c in src:  # new inputs, written eagerly
            c.normal_(generator=torch.Generator(device=gpu).manual_seed(100 + rep))
        for t in [st, st_t] + dst + rot + tok:
            t.zero_()
        g.replay()
        got = snapshot()
        for t in [st, st_t] + dst + rot + tok:
            t.zero_()
        step()
        want = snapshot()
        for i, (a, b) in enumerate(zip(got, want)):
            assert torch.equal(a, b), f"replay {rep}, output {i}"
    assert want[0].any() and want[1].any() and want[-1].any()
    # host tables under capture are refused: their upload would be replayed
    # from a pinned buffer that torch reuses
    g2 = torch.cuda.CUDAGraph()
    with pytest.raises(ValueError, match="graph capture"):
        with torch.cuda.graph(g2):
            ops.gather(table_s, wl.page_ids, wl.slot_offsets, st)


def _random_cases(n, seed):
    rng = np.random.default_rng(seed)
    cases = []
    while len(cases) < n:
        dt = ["bf16", "fp16", "e4m3", "e5m2"][rng.integers(4)]
        e = 1 if dt in FP8 else 2
        ve = 16 if e == 1 else 8
        D = int(rng.choice([64, 80, 96, 128, 192, 256]))
        H = int(rng.choice([1, 2, 3, 4, 8]))
        bs = int(rng.choice([1, 4, 8, 16, 32]))
        style = "gptj" if rng.random() < 0.25 else "neox"
        u = rng.random()
        R = D if u < 0.6 else D // 2 if u < 0.8 else 2 * int(rng.integers(1, D // 2 + 1))
        if (R // 2) % ve or (R % ve if style == "gptj" else 0) or ((D - R) * e) % 16:
            if rng.random() < 0.5:  # keep some widths for the LDS kernel, skip others
                continue
        if (bs * H * D * e) % 16:
            continue
        cases.append((dt, D, H, bs, style, R, int(rng.integers(1, 6)), int(rng.integers(1 << 30))))
    return cases


# DSR_TEST_RANDOM_CASES widens the draw for longer runs (default 40 / 20).
_N_RANDOM = int(__import__("os").environ.get("DSR_TEST_RANDOM_CASES", "40"))


@pytest.mark.parametrize("dt,D,H,bs,style,R,L,seed", _random_cases(_N_RANDOM, 2024))
def test_random_geometry_parity(gpu, dt, D, H, bs, style, R, L, seed):
    """Seeded random geometries (page and row sizes of every kernel class,
    partial rotary, gptj) through gather, scatter and re-rotation, against
    the oracle."""
    print(f"case: random {dt} D{D} H{H} bs{bs} {style} R{R} L{L} seed{seed}", flush=True)
    shape = KVShape(L, H, D, bs, 1 if dt in FP8 else 2)
    rng = np.random.default_rng(seed)
    nb = int(rng.integers(8, 40))
    n = int(rng.integers(1, nb))
    src = rand_caches(shape, nb, dt, gpu, seed=seed % 1000, scale=40.0 if dt in FP8 else 1.0)
    ids = rng.permutation(nb)[:n].astype(np.int32)
    offs = rng.permutation(n).astype(np.int64) * shape.slot_bytes
    st = torch.zeros(n * shape.slot_bytes, dtype=torch.uint8, device=gpu)
    ops.gather(ops.LayerTable(src), ids, offs, st)
    host = _np_layers(src, dt)
    ref = np.zeros(n * shape.slot_bytes, dtype=np.uint8)
    oracle.gather(host, ids, offs, ref, shape.layer_bytes)
    torch.cuda.synchronize()
    assert np.array_equal(st.cpu().numpy(), ref)
    dst_ids = rng.permutation(nb)[:n].astype(np.int32)
    deltas = rng.integers(-4000, 32768, size=n) * (rng.random(n) < 0.8)
    ridx, uniq = position.page_rope_index([1] * n, deltas)
    tabs = position.delta_tables(uniq or [0], R, 500000.0, device=gpu)
    ks_np = (rng.random(L).astype(np.float32) * 0.5 + 0.01) if dt in FP8 else None
    ks = torch.from_numpy(ks_np).to(gpu) if ks_np is not None else None
    dst = [torch.zeros_like(c) for c in src]
    ops.scatter(ops.LayerTable(dst), dst_ids, offs, st)
    rot = [torch.zeros_like(c) for c in src]
    ops.scatter_rerotate(ops.LayerTable(rot), dst_ids, offs, st, tabs, ridx, rot_dim=R,
                         style=style, k_scale=ks)
    dref = [np.zeros_like(h) for h in host]
    oracle.scatter(dref, dst_ids, offs, ref, shape.layer_bytes)
    rref = [np.zeros_like(h) for h in host]
    d = np.asarray(deltas, np.int64)
    oracle.scatter_rerotate(rref, dst_ids, offs, ref, shape.layer_bytes, dtype=ORC_DT[dt],
                            rot_dim=R, style=0 if style == "neox" else 1,
                            stored_pos=np.zeros(n, np.int64), new_pos=d, rotate=d != 0,
                            theta=500000.0, k_scale=ks_np)
    torch.cuda.synchronize()
    for l in range(L):
        assert np.array_equal(to_bits_np(dst[l], dt), dref[l]), f"scatter layer {l}"
        got = to_bits_np(rot[l], dt)
        assert np.array_equal(got[1], rref[l][1]), f"V layer {l}"
        ok, msg = rotation_within_tolerance(got[0], rref[l][0], dt)
        assert ok, f"K layer {l}: {msg}"
    # the same data as split-x pages (3-D caches), where the geometry allows:
    # bit-identical to the token-major result after the layout permutation
    e = shape.elem_bytes
    X = 16 // e
    ve = X
    whole = ((R // 2) % ve == 0 if style == "neox" else R % ve == 0) and ((D - R) * e) % 16 == 0
    if whole and D % X == 0:
        tdt = rot[0].dtype
        st_kx = (st.view(tdt).view(n, L, 2, bs, H, D // X, X).permute(0, 1, 2, 4, 5, 3, 6)
                 .contiguous().view(-1).view(torch.uint8))
        kx = [torch.zeros((2, nb, bs * H * D), dtype=tdt, device=gpu) for _ in range(L)]
        ops.scatter_rerotate(ops.LayerTable(kx, block_size=bs, head_dim=D), dst_ids, offs, st_kx,
                             tabs, ridx, rot_dim=R, style=style, k_scale=ks)
        torch.cuda.synchronize()
        for l in range(L):
            back = kx[l].view(2, nb, H, D // X, bs, X).permute(0, 1, 4, 2, 3, 5).reshape(
                2, nb, bs, H, D)
            assert torch.equal(back.view(torch.uint8), rot[l].view(torch.uint8)), \
                f"split-x layer {l}"
    # head-major (HND) pages holding the same values: the same records, and
    # (where the contig / grouped kernels apply) the same re-rotated bits
    if H > 1 and bs > 1:
        def hnd_like(cs):
            out = []
            for c in cs:
                m = torch.empty((2, nb, H, bs, D), dtype=c.dtype, device=gpu)
                v = m.permute(0, 1, 3, 2, 4)
                v.copy_(c)
                out.append(v)
            return out
        st_h = torch.zeros_like(st)
        ops.gather(ops.LayerTable(hnd_like(src)), ids, offs, st_h)
        torch.cuda.synchronize()
        assert torch.equal(st_h, st), "head-major gather"
        hv = (R // 2) * e // 16 if style == "neox" else 0
        row_vecs = D * e // 16
        if whole and (style == "gptj" or (0 < hv <= 32 and hv & (hv - 1) == 0
                                          and row_vecs % (2 * hv) == 0)):
            hr = hnd_like([torch.zeros_like(c) for c in src])
            ops.scatter_rerotate(ops.LayerTable(hr), dst_ids, offs, st, tabs, ridx, rot_dim=R,
                                 style=style, k_scale=ks)
            torch.cuda.synchronize()
            for l in range(L):
                assert torch.equal(hr[l].contiguous().view(torch.uint8),
                                   rot[l].view(torch.uint8)), f"head-major layer {l}"


@pytest.mark.parametrize("dt,D,H,bs,style,R,L,seed", _random_cases(max(1, _N_RANDOM // 2), 77))
def test_random_geometry_slots_parity(gpu, dt, D, H, bs, style, R, L, seed):
    """Token-granular gather / scatter on random geometries and random
    slot mappings (ragged requests, partial pages, padding) vs the oracle."""
    print(f"case: random slots {dt} D{D} H{H} bs{bs} L{L} seed{seed}", flush=True)
    shape = KVShape(L, H, D, bs, 1 if dt in FP8 else 2)
    rng = np.random.default_rng(seed)
    nb = int(rng.integers(16, 64))
    toks = [int(x) for x in rng.integers(1, 6 * bs, size=int(rng.integers(1, 5)))]
    pages = [(t + bs - 1) // bs for t in toks]
    if sum(pages) > nb:
        pytest.skip("pool too small for this draw")
    perm = rng.permutation(nb).astype(np.int64)
    tables, k = [], 0
    for p in pages:
        tables.append(perm[k:k + p].tolist())
        k += p
    row = H * D * shape.elem_bytes
    sm = ops.slot_mapping_for(tables, toks, bs)
    ro = ops.token_row_offsets(toks, shape.slot_bytes, bs, row)
    sm[rng.random(sm.size) < 0.1] = -1  # padding
    src = rand_caches(shape, nb, dt, gpu, seed=seed % 997)
    st = torch.zeros(sum(pages) * shape.slot_bytes, dtype=torch.uint8, device=gpu)
    ops.gather_slots(ops.LayerTable(src), sm, ro, st)
    host = _np_layers(src, dt)
    ref = np.zeros(st.numel(), dtype=np.uint8)
    oracle.gather_slots(host, sm, ro, ref, shape.layer_bytes)
    dst = [torch.zeros_like(c) for c in src]
    ops.scatter_slots(ops.LayerTable(dst), sm, ro, st)
    dref = [np.zeros_like(h) for h in host]
    oracle.scatter_slots(dref, sm, ro, ref, shape.layer_bytes)
    torch.cuda.synchronize()
    assert np.array_equal(st.cpu().numpy(), ref)
    for l in range(L):
        assert np.array_equal(to_bits_np(dst[l], dt), dref[l]), f"layer {l}"


def _token_tables(deltas, rot_dim, gpu, theta=500000.0):
    """rope_idx per token (-1 where the delta is 0) and the delta tables."""
    d = np.asarray(deltas, np.int64)
    uniq = sorted({int(x) for x in d if x})
    idx = np.array([uniq.index(int(x)) if x else -1 for x in d], np.int64)
    return idx, position.delta_tables(uniq or [0], rot_dim, theta, device=gpu)


@pytest.mark.parametrize("form", ["host", "device"])
@pytest.mark.parametrize("dt,style,D,R,H,bs", [
    ("bf16", "neox", 128, 128, 8, 16),
    ("bf16", "neox", 128, 96, 2, 16),   # partial rotary, half of 6 vectors
    ("bf16", "gptj", 64, 32, 4, 8),
    ("fp16", "neox", 256, 128, 1, 16),
    ("fp16", "gptj", 128, 128, 8, 32),
    ("e4m3", "neox", 128, 128, 8, 16),
    ("e4m3", "gptj", 128, 64, 4, 16),
    ("e5m2", "neox", 128, 64, 8, 16),
    ("e5m2", "gptj", 256, 256, 2, 16),
])
def test_slots_rerotate_matches_oracle(gpu, dt, style, D, R, H, bs, form):
    """Token-form load with per-request deltas (ragged requests, partial
    pages, padding, requests kept at their position) against the oracle:
    V bit-exact, K within the rotation tolerance. Host tables send whole
    pages through the page re-rotation; device tables take the token kernel
    for every token."""
    print(f"case: slots rerotate {dt} {style} D{D} R{R} H{H} bs{bs} {form}", flush=True)
    L = 3
    shape = KVShape(L, H, D, bs, 1 if dt in FP8 else 2)
    rng = np.random.default_rng(D * 7 + R + H)
    toks = [int(x) for x in rng.integers(1, 5 * bs, size=5)]
    pages = [(t + bs - 1) // bs for t in toks]
    nb = sum(pages) + 7
    perm = rng.permutation(nb).astype(np.int64)
    tables, k = [], 0
    for p in pages:
        tables.append(perm[k:k + p].tolist())
        k += p
    row = H * D * shape.elem_bytes
    sm = ops.slot_mapping_for(tables, toks, bs)
    ro = ops.token_row_offsets(toks, shape.slot_bytes, bs, row)
    sm[rng.random(sm.size) < 0.1] = -1
    req_delta = [0, 517, -3000, 32767, 1]
    tok_delta = np.repeat(np.asarray(req_delta, np.int64), toks)
    ridx, tabs = _token_tables(tok_delta, R, gpu)
    src = rand_caches(shape, nb, dt, gpu, seed=11, scale=40.0 if dt in FP8 else 1.0)
    st = torch.zeros(sum(pages) * shape.slot_bytes, dtype=torch.uint8, device=gpu)
    ops.gather_slots(ops.LayerTable(src), ops.slot_mapping_for(tables, toks, bs), ro, st)
    ks_np = (rng.random(L).astype(np.float32) * 0.5 + 0.01) if dt in FP8 else None
    ks = torch.from_numpy(ks_np).to(gpu) if ks_np is not None else None
    dst = rand_caches(shape, nb, dt, gpu, seed=12)
    dref = [to_bits_np(c, dt) for c in dst]
    if form == "device":
        ops.scatter_slots_rerotate(ops.LayerTable(dst), torch.from_numpy(sm).to(gpu),
                                   torch.from_numpy(ro).to(gpu), st, tabs,
                                   torch.as_tensor(np.asarray(ridx, np.int32), device=gpu), rot_dim=R,
                                   style=style, k_scale=ks)
    else:
        ops.scatter_slots_rerotate(ops.LayerTable(dst), sm, ro, st, tabs, ridx, rot_dim=R,
                                   style=style, k_scale=ks)
    oracle.scatter_slots_rerotate(
        dref, sm, ro, st.cpu().numpy(), shape.layer_bytes, dtype=ORC_DT[dt], rot_dim=R,
        style=0 if style == "neox" else 1, stored_pos=np.zeros(sm.size, np.int64),
        new_pos=tok_delta, rotate=tok_delta != 0, theta=500000.0, k_scale=ks_np)
    torch.cuda.synchronize()
    for l in range(L):
        got = to_bits_np(dst[l], dt)
        assert np.array_equal(got[1], dref[l][1]), f"V layer {l}"
        ok, msg = rotation_within_tolerance(got[0], dref[l][0], dt)
        assert ok, f"K layer {l}: {msg}"


@pytest.mark.parametrize("dt,style,R", [("bf16", "neox", 128), ("e4m3", "gptj", 64),
                                        ("fp16", "neox", 64)])
def test_slots_rerotate_equals_page_rerotate(gpu, dt, style, R):
    """On whole pages the token form writes the same bits as the page form
    (same tables, same fp32 arithmetic), including grouped layers with a
    layer that has no RoPE."""
    print(f"case: slots rerotate == pages {dt} {style} R{R}", flush=True)
    L, bs = 4, 16
    shape = KVShape(L, 8, 128, bs, 1 if dt in FP8 else 2)
    rng = np.random.default_rng(5)
    n, nb = 9, 24
    src = rand_caches(shape, nb, dt, gpu, seed=3, scale=40.0 if dt in FP8 else 1.0)
    offs = np.arange(n, dtype=np.int64) * shape.slot_bytes
    st = torch.zeros(n * shape.slot_bytes, dtype=torch.uint8, device=gpu)
    ops.gather(ops.LayerTable(src), rng.permutation(nb)[:n].astype(np.int32), offs, st)
    ids = rng.permutation(nb)[:n].astype(np.int64)
    deltas = np.asarray([0, 9, 9, -77, 4000, 4000, 4000, 0, 123], np.int64)
    ridx_p, uniq = position.page_rope_index([1] * n, deltas)
    thetas = (500000.0, 10000.0)
    tabs = torch.stack([position.delta_tables(uniq, R, t, device=gpu) for t in thetas])
    group = torch.tensor([0, 1, -1, 0], dtype=torch.int32, device=gpu)
    ks = torch.full((L,), 0.37, dtype=torch.float32, device=gpu) if dt in FP8 else None
    pg = [torch.zeros_like(c) for c in src]
    ops.scatter_rerotate(ops.LayerTable(pg), ids.astype(np.int32), offs, st, tabs, ridx_p,
                         rot_dim=R, style=style, k_scale=ks, layer_group=group)
    sm = (ids[:, None] * bs + np.arange(bs)[None, :]).reshape(-1)
    row = shape.num_heads * shape.head_dim * shape.elem_bytes
    ro = (offs[:, None] + np.arange(bs)[None, :] * row).reshape(-1)
    ridx_t = np.repeat(np.asarray(ridx_p, np.int64), bs)
    # device tables: the token kernel on every token (host tables would send
    # these whole pages to the page kernel)
    tk = [torch.zeros_like(c) for c in src]
    ops.scatter_slots_rerotate(ops.LayerTable(tk), torch.from_numpy(sm).to(gpu),
                               torch.from_numpy(ro).to(gpu), st, tabs,
                               torch.from_numpy(ridx_t.astype(np.int32)).to(gpu), rot_dim=R,
                               style=style, k_scale=ks, layer_group=group)
    torch.cuda.synchronize()
    for l in range(L):
        assert torch.equal(tk[l].view(torch.uint8), pg[l].view(torch.uint8)), f"layer {l}"


def test_slots_rerotate_rejects_unsupported_heads(gpu):
    """Heads that are not a power-of-two number of 16-byte vectors, or a
    rotary half wider than 128 pairs, are refused."""
    print("case: slots rerotate shape errors", flush=True)
    shape = KVShape(1, 2, 96, 16, 2)  # 12 vectors per head
    caches = rand_caches(shape, 4, "bf16", gpu, seed=1)
    st = torch.zeros(shape.slot_bytes, dtype=torch.uint8, device=gpu)
    tabs = position.delta_tables([5], 96, device=gpu)
    with pytest.raises(DaserKVError):
        ops.scatter_slots_rerotate(ops.LayerTable(caches), [0], [0], st, tabs, [0])
    shape = KVShape(1, 1, 512, 16, 2)  # rot_dim 512 > 256
    caches = rand_caches(shape, 2, "bf16", gpu, seed=1)
    st = torch.zeros(shape.slot_bytes, dtype=torch.uint8, device=gpu)
    tabs = position.delta_tables([5], 512, device=gpu)
    with pytest.raises(DaserKVError):
        ops.scatter_slots_rerotate(ops.LayerTable(caches), [0], [0], st, tabs, [0])


@pytest.mark.parametrize("heads,head_dim,dt", [(8, 128, "bf16"), (1, 128, "bf16"),
                                              (8, 128, "e4m3")])
def test_shared_records_hint_does_not_change_results(gpu, heads, head_dim, dt):
    """DSR_REROTATE_SHARED_RECORDS only reshapes the launch: several pages
    reading the same records give the same bits with and without it (token-
    major and split-x pages), and match the oracle."""
    print(f"case: shared-records hint H{heads} D{head_dim} {dt}", flush=True)
    shape = KVShape(3, heads, head_dim, 16, 1 if dt in FP8 else 2)
    rng = np.random.default_rng(4)
    n_src, n = 3, 12
    nb = n + 4
    src = rand_caches(shape, nb, dt, gpu, seed=61)
    recs = torch.zeros(n_src * shape.slot_bytes, dtype=torch.uint8, device=gpu)
    ops.gather(ops.LayerTable(src), [1, 5, 7], np.arange(n_src) * shape.slot_bytes, recs)
    offs = (np.arange(n) % n_src).astype(np.int64) * shape.slot_bytes  # each record 4 times
    page_ids = rng.permutation(nb)[:n].astype(np.int32)
    ridx = (np.arange(n) % 2).astype(np.int32)
    tabs = position.delta_tables([77, 30001], head_dim, 500000.0, device=gpu)
    ks = torch.full((3,), 0.05, dtype=torch.float32, device=gpu) if dt in FP8 else None
    outs = []
    for flat in (False, True):
        for hint in (False, True):
            dst = rand_caches(shape, nb, dt, gpu, seed=62)
            caches = [c.reshape(2, nb, -1) for c in dst] if flat else dst
            geo = dict(block_size=16, head_dim=head_dim) if flat else {}
            ops.scatter_rerotate(ops.LayerTable(caches, **geo), page_ids, offs, recs, tabs, ridx,
                                 k_scale=ks, shared_records=hint)
            outs.append([to_bits_np(c, dt) for c in dst])
    torch.cuda.synchronize()
    for l in range(3):
        assert np.array_equal(outs[0][l], outs[1][l]), f"layer {l}: token-major"
        assert np.array_equal(outs[2][l], outs[3][l]), f"layer {l}: split-x"
    ref = [to_bits_np(c, dt) for c in rand_caches(shape, nb, dt, gpu, seed=62)]
    delta = np.where(ridx == 0, 77, 30001)
    oracle.scatter_rerotate(ref, page_ids, offs, recs.cpu().numpy(), shape.layer_bytes,
                            dtype=ORC_DT[dt], rot_dim=head_dim, style=0,
                            stored_pos=np.zeros(n, np.int64), new_pos=delta,
                            rotate=np.ones(n, bool), theta=500000.0,
                            k_scale=None if ks is None else np.full(3, 0.05, np.float32))
    for l in range(3):
        assert np.array_equal(outs[0][l][1], ref[l][1])
        ok, msg = rotation_within_tolerance(outs[0][l][0][page_ids], ref[l][0][page_ids], dt)
        assert ok, f"layer {l}: {msg}"


@pytest.mark.parametrize("heads,head_dim,dt", [(1, 128, "bf16"), (1, 128, "e4m3"),
                                              (2, 64, "bf16")])
def test_rerotate_contig_override_on_small_pages(gpu, tuning, heads, head_dim, dt):
    """Small pages default to the grouped kernel; the "contig" rot_kernel override runs
    the one-unit contig kernel instead, which must then be launched with one
    unit per workgroup (every page written, same bits as the grouped
    kernel)."""
    print(f"case: contig override H{heads} D{head_dim} {dt}", flush=True)
    shape, dst, dst_ref, page_ids, _ = _rerotate_case(gpu, dt, "neox", head_dim, head_dim,
                                                      heads=heads, layers=3, seed=8)
    tuning("rot_kernel", "contig")
    shape2, dst2, _, page_ids2, _ = _rerotate_case(gpu, dt, "neox", head_dim, head_dim,
                                                   heads=heads, layers=3, seed=8)
    torch.cuda.synchronize()
    assert np.array_equal(page_ids, page_ids2)
    for a, b in zip(dst, dst2):
        assert torch.equal(a.view(torch.uint8), b.view(torch.uint8))


@pytest.mark.parametrize("heads,head_dim,dt,kernel", [
    (8, 128, "bf16", None),    # grouped kernel, one unit per workgroup
    (1, 128, "bf16", None),    # grouped, several units per workgroup
    (8, 128, "e4m3", None),    # contig kernel
    (8, 128, "e5m2", None),    # contig kernel, e5m2
    (1, 128, "e5m2", None),    # grouped, e5m2
    (4, 96, "bf16", None),     # row-aligned kernel
    (4, 96, "bf16", "pairs"),  # pair-task kernel
    (16, 128, "bf16", None),   # 64 KiB pages: contig kernel in rounds
    (4, 96, "bf16", "lds24"),  # rotary width 24 of 96: the LDS kernel
])
def test_rerotate_per_layer_groups(gpu, tuning, heads, head_dim, dt, kernel):
    """Layers with different RoPE bases (local / global attention) and layers
    without RoPE: layer_group picks each layer's table block; group -1
    copies K. Each layer matches the oracle run with its own base."""
    print(f"case: rerotate layer groups H{heads} D{head_dim} {dt} {kernel}", flush=True)
    rot = head_dim
    if kernel == "lds24":
        rot = 24
    elif kernel:
        tuning("rot_kernel", kernel)
    L = 6
    groups = np.array([0, 1, -1, 0, 1, -1], np.int32)
    thetas = [10000.0, 1000000.0]
    shape = KVShape(L, heads, head_dim, 16, 1 if dt in FP8 else 2)
    rng = np.random.default_rng(heads * 1000 + head_dim)
    nb, n = 24, 10
    src = rand_caches(shape, nb, dt, gpu, seed=91, scale=40.0 if dt in FP8 else 1.0)
    st = torch.zeros(n * shape.slot_bytes, dtype=torch.uint8, device=gpu)
    offs = np.arange(n, dtype=np.int64) * shape.slot_bytes
    ops.gather(ops.LayerTable(src), rng.permutation(nb)[:n].astype(np.int32), offs, st)
    deltas = rng.integers(1, 32768, size=n) * (np.arange(n) % 4 != 0)  # some pages unmoved
    ridx, uniq = position.page_rope_index([1] * n, deltas)
    tabs = torch.stack([position.delta_tables(uniq, rot, t, device=gpu) for t in thetas])
    ks_np = (rng.random(L).astype(np.float32) * 0.5 + 0.01) if dt in FP8 else None
    ks = torch.from_numpy(ks_np).to(gpu) if ks_np is not None else None
    dst_ids = rng.permutation(nb)[:n].astype(np.int32)
    out = [torch.zeros_like(c) for c in src]
    ops.scatter_rerotate(ops.LayerTable(out), dst_ids, offs, st, tabs, ridx, k_scale=ks,
                         layer_group=groups, rot_dim=rot)
    recs = st.cpu().numpy()
    d = np.asarray(deltas, np.int64)
    torch.cuda.synchronize()
    for l in range(L):
        ref = [np.zeros_like(to_bits_np(src[l], dt))]
        g = groups[l]
        oracle.scatter_rerotate(ref, dst_ids, offs, recs, shape.layer_bytes, dtype=ORC_DT[dt],
                                rot_dim=rot, style=0, stored_pos=np.zeros(n, np.int64),
                                new_pos=d, rotate=(d != 0) & (g >= 0),
                                theta=thetas[max(g, 0)], k_scale=ks_np, layer0=l)
        got = to_bits_np(out[l], dt)
        assert np.array_equal(got[1], ref[0][1]), f"V layer {l}"
        if g < 0:
            assert np.array_equal(got[0], ref[0][0]), f"no-RoPE layer {l} must be a copy"
        ok, msg = rotation_within_tolerance(got[0], ref[0][0], dt)
        assert ok, f"K layer {l} (group {g}): {msg}"


def test_concurrent_streams_match_sequential(gpu):
    """The entry points hold no state between calls: gathers and re-rotating
    scatters issued on two streams at once write what the same calls write
    one after the other."""
    print("case: two streams", flush=True)
    shape = KVShape(4, 8, 128, 16, 2)
    wl = workloads.ragged(shape, 6, 200, 900, seed=15, num_blocks=512)
    src = rand_caches(shape, wl.num_blocks, "bf16", gpu, seed=95)
    table = ops.LayerTable(src)
    halves = np.array_split(np.arange(wl.n_pages), 2)
    tabs = position.delta_tables([77, 20001], 128, 500000.0, device=gpu)
    ridx = (np.arange(wl.n_pages) % 3 - 1).astype(np.int32)

    def work(dsts, outs, streams):
        for h, (idx, s) in enumerate(zip(halves, streams)):
            with torch.cuda.stream(s):
                ops.gather(table, wl.page_ids[idx], wl.slot_offsets[idx], outs[h])
                ops.scatter_rerotate(ops.LayerTable(dsts[h]), wl.page_ids[idx],
                                     wl.slot_offsets[idx], outs[h], tabs, ridx[idx])

    def fresh():
        return ([[torch.zeros_like(c) for c in src] for _ in range(2)],
                [torch.zeros(wl.staging_bytes, dtype=torch.uint8, device=gpu)
                 for _ in range(2)])

    seq_d, seq_o = fresh()
    cur = torch.cuda.current_stream(gpu)
    work(seq_d, seq_o, [cur, cur])
    torch.cuda.synchronize()
    par_d, par_o = fresh()
    streams = [torch.cuda.Stream(gpu), torch.cuda.Stream(gpu)]
    for s in streams:
        s.wait_stream(cur)
    work(par_d, par_o, streams)
    torch.cuda.synchronize()
    for h in range(2):
        assert torch.equal(seq_o[h], par_o[h])
        for a, b in zip(seq_d[h], par_d[h]):
            assert torch.equal(a, b)


# ---------------------------------------------------------------------------
# 3-D caches: byte copies for any page layout, re-rotation of split-x K pages


def _flat_caches(shape, nb, dt, gpu, seed, scale=1.0):
    """(2, NB, block_size * H * D) caches, as vLLM's PagedAttention backend
    allocates them."""
    return [c.reshape(2, nb, -1) for c in rand_caches(shape, nb, dt, gpu, seed, scale)]


def test_flat_cache_copies_bit_exact(gpu):
    """Gather/scatter move kv[:, b] of a 3-D cache as bytes, like the
    reference's copy_ of any cache shape; no head geometry is needed."""
    print("case: 3-D cache copies", flush=True)
    shape = KVShape(3, 2, 64, 16, 2)
    wl = workloads.ragged(shape, 4, 1, 120, seed=4, pool_slack=1.5)
    caches = _flat_caches(shape, wl.num_blocks, "bf16", gpu, seed=12)
    staging, ref = _gather_both(wl, caches, "bf16", gpu)
    torch.cuda.synchronize()
    assert np.array_equal(staging.cpu().numpy(), ref)
    dst = [torch.zeros_like(c) for c in caches]
    ops.scatter(ops.LayerTable(dst), wl.page_ids, wl.slot_offsets, staging)
    torch.cuda.synchronize()
    ids = torch.from_numpy(wl.page_ids.astype(np.int64)).to(gpu)
    for l in range(shape.num_layers):
        assert torch.equal(dst[l][:, ids], caches[l][:, ids])
    table = ops.LayerTable(caches)
    assert table.layout.k_layout == "kx" and not table.layout.has_geometry
    tabs = position.delta_tables([3], 64, device=gpu)
    with pytest.raises(ValueError):  # no head geometry: re-rotation refused
        ops.scatter_rerotate(table, wl.page_ids[:1], wl.slot_offsets[:1], staging, tabs, [0])
    with pytest.raises(ValueError):  # no token-major rows: the token form refused
        ops.gather_slots(ops.LayerTable(caches, block_size=16, head_dim=64), [0], [0], staging)


@pytest.mark.parametrize("dt,style,heads,head_dim,rot_dim", [
    ("bf16", "neox", 4, 128, 128),
    ("bf16", "neox", 1, 128, 64),    # partial rotary: tail vectors copied
    ("bf16", "gptj", 2, 64, 64),
    ("fp16", "neox", 8, 128, 128),
    ("e4m3", "neox", 2, 128, 128),
    ("e4m3", "gptj", 1, 128, 96),
    ("e5m2", "neox", 2, 128, 128),
    ("bf16", "neox", 3, 96, 96),     # 12-vector columns: the pair-task kernel
])
@pytest.mark.parametrize("kernel", ["auto", "pairs"])
def test_rerotate_kx_layout_matches_oracle(gpu, tuning, dt, style, heads, head_dim,
                                           rot_dim, kernel):
    """Split-x K pages (vLLM PagedAttention layout) re-rotated by the kernel
    equal the oracle's token-major re-rotation of the same pages moved into
    [block_size][H][D] order and back (oracle.kx_to_nhd, pinned by a brute
    force index test); V and unrotated pages bit-exact."""
    print(f"case: kx re-rotate {dt} {style} H{heads} D{head_dim} R{rot_dim} {kernel}",
          flush=True)
    if kernel == "pairs":
        tuning("rot_kernel", "pairs")
    bs, L = 16, 3
    shape = KVShape(L, heads, head_dim, bs, 1 if dt in FP8 else 2)
    rng = np.random.default_rng(17)
    deltas = (0, 5, 4097, 32767)
    chunk_pages = [2, 1, 3, 2]
    n = sum(chunk_pages)
    nb = n + 5
    geo = dict(block_size=bs, head_dim=head_dim)
    src = _flat_caches(shape, nb, dt, gpu, seed=21, scale=2.0)
    staging = torch.zeros(n * shape.slot_bytes, dtype=torch.uint8, device=gpu)
    offs = np.arange(n, dtype=np.int64) * shape.slot_bytes
    ops.gather(ops.LayerTable(src, **geo), rng.permutation(nb)[:n].astype(np.int32), offs,
               staging)
    dst = _flat_caches(shape, nb, dt, gpu, seed=22)
    before = [to_bits_np(c, dt) for c in dst]
    page_ids = rng.permutation(nb)[:n].astype(np.int32)
    ridx, uniq = position.page_rope_index(chunk_pages, deltas)
    tabs = position.delta_tables(uniq, rot_dim, 500000.0, device=gpu)
    ks_np = k_scale = None
    if dt in FP8:
        ks_np = rng.random(L).astype(np.float32) * 0.5 + 0.01
        k_scale = torch.from_numpy(ks_np).to(gpu)
    table = ops.LayerTable(dst, **geo)
    assert table.layout.k_layout == "kx" and table.layout.num_heads == heads
    ops.scatter_rerotate(table, page_ids, offs, staging, tabs, ridx, rot_dim=rot_dim,
                         style=style, k_scale=k_scale)
    # oracle in token-major order: permute caches and records, rotate, compare
    to_nhd = lambda a: oracle.kx_to_nhd(a, bs, heads, head_dim)  # noqa: E731
    ref = [np.ascontiguousarray(to_nhd(b)) for b in before]
    el = np.uint8 if dt in FP8 else np.uint16
    recs = staging.cpu().numpy().view(el).reshape(n, L, 2, -1)
    recs_nhd = np.ascontiguousarray(to_nhd(recs)).reshape(-1).view(np.uint8)
    page_delta = np.repeat(np.asarray(deltas, np.int64), chunk_pages)
    oracle.scatter_rerotate(
        ref, page_ids, offs, recs_nhd, shape.layer_bytes, dtype=ORC_DT[dt], rot_dim=rot_dim,
        style=0 if style == "neox" else 1, stored_pos=np.zeros(n, np.int64),
        new_pos=page_delta, rotate=page_delta != 0, theta=500000.0, k_scale=ks_np)
    torch.cuda.synchronize()
    touched = np.zeros(nb, bool)
    touched[page_ids] = True
    for l in range(L):
        got = to_nhd(to_bits_np(dst[l], dt))
        assert np.array_equal(got[1], ref[l][1]), f"layer {l}: V"
        assert np.array_equal(got[:, ~touched], ref[l][:, ~touched]), f"layer {l}: untouched"
        ok, msg = rotation_within_tolerance(got[0][page_ids], ref[l][0][page_ids], dt)
        assert ok, f"layer {l}: {msg}"
        still = page_ids[page_delta == 0]
        assert np.array_equal(got[0][still], ref[l][0][still]), f"layer {l}: delta 0 copy"


# ---------------------------------------------------------------------------
# head-major (HND) cache pages: records in token-major order


def _hnd_caches(shape, nb, dt, gpu, seed, scale=1.0):
    """(2, NB, bs, H, D) views of head-major memory (2, NB, H, bs, D), holding
    the same logical values as rand_caches with the same seed."""
    out = []
    for c in rand_caches(shape, nb, dt, gpu, seed, scale):
        m = torch.empty((2, nb, shape.num_heads, shape.block_size, shape.head_dim),
                        dtype=c.dtype, device=gpu)
        v = m.permute(0, 1, 3, 2, 4)
        v.copy_(c)
        out.append(v)
    return out


@pytest.mark.parametrize("heads,head_dim,bs,dt", [
    (8, 128, 16, "bf16"), (2, 64, 16, "bf16"), (4, 128, 32, "e4m3"), (3, 96, 16, "bf16"),
    (2, 32, 16, "bf16"),   # 2 KiB pages: the grouped copies
    (4, 64, 16, "e4m3"),   # 4 KiB e4m3: grouped scatter, one-unit gather
])
def test_hnd_copies_match_oracle(gpu, heads, head_dim, bs, dt):
    """Gather from head-major pages writes the records of the logical page
    (the reference's reshape(-1) of kv[:, b]); scatter writes them back."""
    print(f"case: hnd copies H{heads} D{head_dim} bs{bs} {dt}", flush=True)
    shape = KVShape(3, heads, head_dim, bs, 1 if dt in FP8 else 2)
    wl = workloads.ragged(shape, 4, 1, 200, seed=5, pool_slack=1.5)
    caches = _hnd_caches(shape, wl.num_blocks, dt, gpu, seed=70)
    table = ops.LayerTable(caches)
    assert table.layout.k_layout == "hnd"
    st = torch.zeros(wl.staging_bytes, dtype=torch.uint8, device=gpu)
    ops.gather(table, wl.page_ids, wl.slot_offsets, st)
    ref = np.zeros(wl.staging_bytes, dtype=np.uint8)
    host = [np.ascontiguousarray(to_bits_np(c, dt)) for c in caches]
    oracle.gather(host, wl.page_ids, wl.slot_offsets, ref, shape.layer_bytes)
    torch.cuda.synchronize()
    assert np.array_equal(st.cpu().numpy(), ref)
    dst = _hnd_caches(shape, wl.num_blocks, dt, gpu, seed=71)
    before = [to_bits_np(c, dt) for c in dst]
    ops.scatter(ops.LayerTable(dst), wl.page_ids, wl.slot_offsets, st)
    dref = [np.ascontiguousarray(b) for b in before]
    oracle.scatter(dref, wl.page_ids, wl.slot_offsets, ref, shape.layer_bytes)
    torch.cuda.synchronize()
    for l in range(3):
        assert np.array_equal(to_bits_np(dst[l], dt), dref[l]), f"layer {l}"
    # the per-layer prepared gather of the connector takes the same route
    st2 = torch.zeros_like(st)
    pg = ops.PreparedGather(table, torch.from_numpy(wl.page_ids).to(gpu),
                            torch.from_numpy(wl.slot_offsets).to(gpu), st2)
    for l in range(3):
        pg(l, 1, torch.cuda.current_stream(gpu).cuda_stream)
    torch.cuda.synchronize()
    assert torch.equal(st, st2)
    with pytest.raises(ValueError):  # the token form needs token-major pages
        ops.gather_slots(table, [0], [0], st)


@pytest.mark.parametrize("heads,head_dim,rot,dt,style", [
    (8, 128, 128, "bf16", "neox"), (2, 64, 64, "bf16", "neox"), (4, 128, 128, "e4m3", "neox"),
    (2, 128, 128, "bf16", "gptj"), (4, 128, 64, "bf16", "neox"),
    (2, 128, 128, "e4m3", "neox"),  # 4 KiB e4m3 pages: grouped
    (4, 128, 128, "e5m2", "gptj"),
    (2, 32, 32, "bf16", "neox"),    # 2 KiB pages: grouped, 16 units per workgroup
    (16, 128, 128, "bf16", "neox"),  # 64 KiB pages: contig in rounds
])
def test_hnd_rerotate_equals_token_major(gpu, heads, head_dim, rot, dt, style):
    """Re-rotation into head-major pages gives, per logical element, exactly
    the bits of the token-major kernel on the same records, and matches the
    oracle."""
    print(f"case: hnd rerotate H{heads} D{head_dim} R{rot} {dt} {style}", flush=True)
    shape, dst, dst_ref, page_ids, deltas = _rerotate_case(gpu, dt, style, head_dim, rot,
                                                           heads=heads, layers=3, seed=9)
    # the same call on head-major caches holding the same initial values
    rng = np.random.default_rng(9)
    chunk_pages = [int(x) for x in rng.integers(1, 4, size=5)]
    n = sum(chunk_pages)
    nb = n + 5
    src_caches = rand_caches(shape, nb, dt, gpu, seed=10)
    staging = torch.zeros(n * shape.slot_bytes, dtype=torch.uint8, device=gpu)
    offs = np.arange(n, dtype=np.int64) * shape.slot_bytes
    ops.gather(ops.LayerTable(src_caches), rng.permutation(nb)[:n].astype(np.int32), offs,
               staging)
    hnd = _hnd_caches(shape, nb, dt, gpu, seed=11)
    ids = rng.permutation(nb)[:n].astype(np.int32)
    assert np.array_equal(ids, page_ids)
    ridx, uniq = position.page_rope_index(chunk_pages, (0, 1, 517, 32767, 123))
    tabs = position.delta_tables(uniq, rot, 500000.0, device=gpu)
    ks = None
    if dt in FP8:
        ks = torch.from_numpy(rng.random(3).astype(np.float32) * 0.5 + 0.01).to(gpu)
    ops.scatter_rerotate(ops.LayerTable(hnd), ids, offs, staging, tabs, ridx, rot_dim=rot,
                         style=style, k_scale=ks)
    torch.cuda.synchronize()
    for l in range(3):
        assert torch.equal(hnd[l].contiguous().view(torch.uint8), dst[l].view(torch.uint8)), \
            f"layer {l}"
        got = to_bits_np(dst[l], dt)
        ok, msg = rotation_within_tolerance(got[0][page_ids], dst_ref[l][0][page_ids], dt)
        assert ok, f"layer {l}: {msg}"


def test_hnd_rerotate_unsupported_width_refused(gpu):
    shape = KVShape(2, 2, 96, 16, 2)
    caches = _hnd_caches(shape, 4, "bf16", gpu, seed=12)
    st = torch.zeros(shape.slot_bytes, dtype=torch.uint8, device=gpu)
    tabs = position.delta_tables([5], 96, device=gpu)
    with pytest.raises(DaserKVError):  # 96-dim neox rows: partners 6 vectors apart
        ops.scatter_rerotate(ops.LayerTable(caches), [1], [0], st, tabs, [0])


@pytest.mark.parametrize("H,D,bs,style,parts", [
    (8, 128, 32, "neox", 0), (8, 256, 16, "neox", 0), (8, 128, 32, "gptj", 0),
    (32, 96, 16, "neox", 0), (32, 96, 16, "neox", 2), (8, 128, 32, "neox", 1),
    (8, 128, 48, "neox", 0), (8, 128, 32, "neox", -64), (32, 96, 16, "neox", -64)])
def test_large_pages_in_parts_match_oracle(gpu, tuning, H, D, bs, style, parts):
    """Pages above 32 KiB move in parts of whole rows, one workgroup each:
    the gather, the streaming scatter, the grouped re-rotation (64 KiB
    pages) and the row-aligned re-rotation (head_dim 96, 96 KiB pages) give
    the oracle's bytes and rotation (parts 0 = the launch policy's choice,
    1 = whole pages; 96 KiB pages at block_size 48; -n: the policy's parts
    with launches cut to n workgroups, so one call runs as many launches)."""
    print(f"case: large pages H{H} D{D} bs{bs} {style} parts={parts}", flush=True)
    if parts > 0:
        tuning("page_parts", parts)
    elif parts < 0:
        tuning("max_wg_per_launch", -parts)
    shape = KVShape(3, H, D, bs, 2)
    wl = workloads.ragged(shape, 5, 30, 900, seed=H + D + bs, pool_slack=1.2)
    caches = rand_caches(shape, wl.num_blocks, "bf16", gpu, seed=71)
    table = ops.LayerTable(caches)
    host = _np_layers(caches, "bf16")
    ref = np.zeros(wl.staging_bytes, dtype=np.uint8)
    oracle.gather(host, wl.page_ids, wl.slot_offsets, ref, shape.layer_bytes)
    st = torch.zeros(wl.staging_bytes, dtype=torch.uint8, device=gpu)
    ops.gather(table, wl.page_ids, wl.slot_offsets, st)
    torch.cuda.synchronize()
    assert np.array_equal(st.cpu().numpy(), ref)
    rng = np.random.default_rng(5)
    dst_ids = rng.permutation(wl.num_blocks)[:wl.n_pages].astype(np.int32)
    deltas = rng.integers(-3000, 30000, size=len(wl.req_pages)) * (rng.random(len(wl.req_pages)) < 0.8)
    ridx, uniq = position.page_rope_index(wl.req_pages, deltas)
    tabs = position.delta_tables(uniq or [0], D, 500000.0, device=gpu)
    dst = [torch.zeros_like(c) for c in caches]
    rot = [torch.zeros_like(c) for c in caches]
    ops.scatter(ops.LayerTable(dst), dst_ids, wl.slot_offsets, st)
    ops.scatter_rerotate(ops.LayerTable(rot), dst_ids, wl.slot_offsets, st, tabs, ridx,
                         style=style)
    dref = [np.zeros_like(h) for h in host]
    oracle.scatter(dref, dst_ids, wl.slot_offsets, ref, shape.layer_bytes)
    rref = [np.zeros_like(h) for h in host]
    d = np.repeat(np.asarray(deltas, np.int64), wl.req_pages)
    oracle.scatter_rerotate(rref, dst_ids, wl.slot_offsets, ref, shape.layer_bytes,
                            dtype=oracle.BF16, rot_dim=D, style=0 if style == "neox" else 1,
                            stored_pos=np.zeros(wl.n_pages, np.int64), new_pos=d, rotate=d != 0,
                            theta=500000.0)
    torch.cuda.synchronize()
    for l in range(shape.num_layers):
        assert np.array_equal(to_bits_np(dst[l], "bf16"), dref[l]), f"scatter layer {l}"
        got = to_bits_np(rot[l], "bf16")
        assert np.array_equal(got[1], rref[l][1]), f"V layer {l}"
        ok, msg = rotation_within_tolerance(got[0], rref[l][0], "bf16")
        assert ok, f"K layer {l}: {msg}"
