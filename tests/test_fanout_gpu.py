"""dsr_scatter_fanout (each shared record read once, written to all of its
destination pages) writes the bytes of the per-page entry points on the
same loads: dsr_scatter_rerotate for the re-rotating form, dsr_scatter for
the plain copy. Called through the C ABI over random geometries; the
per-page entry points are themselves oracle-checked (test_kernels_gpu.py),
and ops' shared-record loads, which take this path, are checked against the
oracle there too."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from daser_amd import _lib, ops, position
from daser_amd.workloads import KVShape
from tests.helpers import TORCH_DT, rand_caches

pytestmark = pytest.mark.gpu

DCODE = {"bf16": 0, "fp16": 1, "e4m3": 2, "e5m2": 3}


def _dev(x, dt=torch.int32):
    return torch.as_tensor(np.ascontiguousarray(x)).to(dt).cuda()


def _case(heads, head_dim, dt, style, rot_dim, groups, n_src, n, seed):
    """Caches (two identical copies), records, per-page tables and the
    fan-out tables of one random load."""
    esize = 1 if dt in ("e4m3", "e5m2") else 2
    shape = KVShape(4, heads, head_dim, 16, esize)
    rng = np.random.default_rng(seed)
    nb = n + 8
    recs = torch.from_numpy(rng.integers(0, 256, n_src * shape.slot_bytes, dtype=np.uint8))
    if esize == 1:  # no NaN codes: NaN bytes are canonicalised, which the test is not about
        recs[(recs & 0x7F) == 0x7F] = 0x11
        if dt == "e5m2":
            recs[(recs & 0x7C) == 0x7C] = 0x21
    else:  # finite 16-bit values
        w = recs.view(torch.int16)
        exp = (w >> (10 if dt == "fp16" else 7)) & (0x1F if dt == "fp16" else 0xFF)
        w[exp == (0x1F if dt == "fp16" else 0xFF)] = 0x3C00 if dt == "fp16" else 0x3F80
    recs = recs.cuda()
    a = rand_caches(shape, nb, dt, "cuda", seed=seed + 1)
    b = [c.clone() for c in a]
    page_ids = rng.permutation(nb)[:n].astype(np.int32)
    src_of = rng.integers(0, n_src, n)
    offs = (src_of * shape.slot_bytes).astype(np.int64)
    n_tables = 5
    ridx = rng.integers(-1, n_tables, n).astype(np.int32)
    tabs = position.delta_tables(list(rng.integers(1, 30000, n_tables)), rot_dim, 500000.0,
                                 device="cuda")
    if groups:
        tabs = torch.stack([tabs, position.delta_tables(list(rng.integers(1, 30000, n_tables)),
                                                        rot_dim, 10000.0, device="cuda")])
        lg = np.array([0, 1, -1, 1], np.int32)
    else:
        lg = None
    ks = torch.tensor([0.03, 0.011, 0.05, 0.02], device="cuda") if esize == 1 else None
    return shape, nb, recs, a, b, page_ids, offs, ridx, tabs, lg, ks, n_tables


def _geometry(shape, cache):
    e = cache.element_size()
    return cache.stride(0) * e, cache.stride(1) * e


@pytest.mark.parametrize("heads,head_dim,dt,style,rot_dim,groups", [
    (8, 128, "bf16", 0, 128, False),   # 32 KiB pages, U = 8
    (4, 128, "bf16", 0, 128, True),    # 16 KiB, layer groups
    (2, 128, "fp16", 1, 128, False),   # 8 KiB, gptj
    (1, 128, "bf16", 0, 64, False),    # 4 KiB, partial rotary
    (8, 128, "e4m3", 0, 128, False),   # 16 KiB e4m3 with scales
    (1, 128, "e5m2", 0, 128, True),    # 2 KiB e5m2, layer groups
    (2, 64, "bf16", 0, 64, False),     # 4 KiB, partner 4 vectors away
    (16, 128, "e4m3", 1, 96, False),   # 32 KiB e4m3, gptj, partial rotary
])
@pytest.mark.parametrize("parts", [1, 2])
def test_fanout_matches_per_page_rerotate(tuning, parts, heads, head_dim, dt, style, rot_dim,
                                          groups):
    print(f"case: fanout H{heads} D{head_dim} {dt} style{style} rot{rot_dim} groups{groups} "
          f"parts{parts}", flush=True)
    tuning("fanout_parts", parts)
    shape, nb, recs, a, b, page_ids, offs, ridx, tabs, lg, ks, n_tables = _case(
        heads, head_dim, dt, style, rot_dim, groups, n_src=7, n=60, seed=heads * 7 + head_dim)
    kv_stride, page_stride = _geometry(shape, a[0])
    lib = _lib.lib()
    stream = torch.cuda.current_stream().cuda_stream
    n_groups = 2 if groups else 0
    lg_d = None if lg is None else _dev(lg)
    ks_p = None if ks is None else ks.data_ptr()
    # per-page entry point on copy a
    base_a = _dev([c.data_ptr() for c in a], torch.int64)
    ids_d, offs_d, ridx_d = _dev(page_ids), _dev(offs, torch.int64), _dev(ridx)
    rc = lib.dsr_scatter_rerotate(
        base_a.data_ptr(), 4, kv_stride, page_stride, shape.page_bytes, nb, ids_d.data_ptr(),
        offs_d.data_ptr(), len(page_ids), recs.data_ptr(), recs.numel(), shape.layer_bytes, 0,
        tabs.data_ptr(), ridx_d.data_ptr(), n_tables, None if lg_d is None else lg_d.data_ptr(),
        n_groups, head_dim, rot_dim, style, DCODE[dt], ks_p, 0, stream)
    _lib.check("dsr_scatter_rerotate", rc)
    # fan-out on copy b
    src, start, dpages, drope = ops.fanout_tables(page_ids, offs, ridx)
    assert start[-1] == len(page_ids) and np.all(np.diff(start) > 0)
    base_b = _dev([c.data_ptr() for c in b], torch.int64)
    src_d, start_d, dp_d, dr_d = (_dev(src, torch.int64), _dev(start), _dev(dpages),
                                  _dev(drope))
    rc = lib.dsr_scatter_fanout(
        base_b.data_ptr(), 4, kv_stride, page_stride, shape.page_bytes, nb, src_d.data_ptr(),
        len(src), start_d.data_ptr(), dp_d.data_ptr(), dr_d.data_ptr(), len(dpages),
        recs.data_ptr(), recs.numel(), shape.layer_bytes, 0, tabs.data_ptr(), n_tables,
        None if lg_d is None else lg_d.data_ptr(), n_groups, head_dim, rot_dim, style,
        DCODE[dt], ks_p, _lib.DSR_K_NHD, 0, 0, stream)
    _lib.check("dsr_scatter_fanout", rc)
    torch.cuda.synchronize()
    for l in range(4):
        assert torch.equal(a[l].view(torch.uint8), b[l].view(torch.uint8)), f"layer {l}"
    # the loads did happen: V of a loaded page is its record's V
    rec = recs.view(-1, 4, 2, shape.page_bytes)
    p = 3
    got = b[1][1, int(page_ids[p])].contiguous().view(torch.uint8).reshape(-1)
    assert torch.equal(got, rec[int(offs[p] // shape.slot_bytes), 1, 1])


@pytest.mark.parametrize("max_wg,parts", [(0, 1), (16, 1), (0, 2), (16, 4)])
def test_fanout_plain_copy_matches_scatter(tuning, max_wg, parts):
    """dst_rope_idx null: the plain load, bit-exact to dsr_scatter, also when
    the sources are split over several launches and units over several
    workgroups."""
    print(f"case: fanout copy max_wg={max_wg} parts={parts}", flush=True)
    if max_wg:
        tuning("max_wg_per_launch", max_wg)
    tuning("fanout_parts", parts)
    shape, nb, recs, a, b, page_ids, offs, *_ = _case(8, 128, "bf16", 0, 128, False,
                                                      n_src=9, n=70, seed=5)
    kv_stride, page_stride = _geometry(shape, a[0])
    lib = _lib.lib()
    stream = torch.cuda.current_stream().cuda_stream
    base_a = _dev([c.data_ptr() for c in a], torch.int64)
    ids_d, offs_d = _dev(page_ids), _dev(offs, torch.int64)
    _lib.check("dsr_scatter", lib.dsr_scatter(
        base_a.data_ptr(), 4, kv_stride, page_stride, shape.page_bytes, nb, ids_d.data_ptr(),
        offs_d.data_ptr(), len(page_ids), recs.data_ptr(), recs.numel(), shape.layer_bytes, 0,
        stream))
    src, start, dpages, _ = ops.fanout_tables(page_ids, offs)
    base_b = _dev([c.data_ptr() for c in b], torch.int64)
    src_d, start_d, dp_d = _dev(src, torch.int64), _dev(start), _dev(dpages)
    _lib.check("dsr_scatter_fanout", lib.dsr_scatter_fanout(
        base_b.data_ptr(), 4, kv_stride, page_stride, shape.page_bytes, nb, src_d.data_ptr(),
        len(src), start_d.data_ptr(), dp_d.data_ptr(), None, len(dpages), recs.data_ptr(),
        recs.numel(), shape.layer_bytes, 0, None, 0, None, 0, 0, 0, 0, 0, None, _lib.DSR_K_NHD,
        0, 0, stream))
    torch.cuda.synchronize()
    for l in range(4):
        assert torch.equal(a[l].view(torch.uint8), b[l].view(torch.uint8)), f"layer {l}"


def test_fanout_through_ops_matches_per_page_path():
    """ops.scatter_rerotate on host tables with shared records takes the
    fan-out path; with the hint off it takes the per-page kernels: same
    bits, including a block listed twice (the last entry kept) and layer
    ranges."""
    print("case: fanout through ops", flush=True)
    shape, nb, recs, a, b, page_ids, offs, ridx, tabs, lg, ks, n_tables = _case(
        8, 128, "bf16", 0, 128, False, n_src=4, n=40, seed=9)
    page_ids = np.append(page_ids, page_ids[5]).astype(np.int32)  # block 5 loaded twice
    offs = np.append(offs, offs[0])
    ridx = np.append(ridx, 2).astype(np.int32)
    for caches, hint in ((a, False), (b, True)):
        ops.scatter_rerotate(ops.LayerTable(caches), page_ids, offs, recs, tabs, ridx,
                             shared_records=hint, layers=(1, 3))
    torch.cuda.synchronize()
    for l in range(4):
        assert torch.equal(a[l].view(torch.uint8), b[l].view(torch.uint8)), f"layer {l}"



def test_token_form_with_shared_chunks_takes_the_fanout():
    """A slot_mapping load in which three requests place the same two cached
    chunks (shared records): its whole pages go through the fan-out, its
    ragged tail through the token kernel; the result equals the per-page
    re-rotation of the same pages (no sharing hint) plus the token kernel."""
    print("case: token form, shared chunks", flush=True)
    shape = KVShape(4, 8, 128, 16, 2)
    bs, row = 16, 8 * 128 * 2
    rng = np.random.default_rng(21)
    n_chunk_pages, n_req = 4, 3
    recs = torch.from_numpy(rng.standard_normal(2 * n_chunk_pages * shape.slot_bytes // 2)
                            .astype(np.float32)).to(torch.bfloat16).view(torch.uint8).cuda()
    nb = 64
    a = rand_caches(shape, nb, "bf16", "cuda", seed=22)
    b = [c.clone() for c in a]
    blocks = rng.permutation(nb)[:n_req * 2 * n_chunk_pages].reshape(n_req, -1)
    tok_per_req = 2 * n_chunk_pages * bs - 5  # the last page ragged
    sm, ro, ri = [], [], []
    for r in range(n_req):
        t = np.arange(tok_per_req)
        sm.append(blocks[r][t // bs] * bs + t % bs)
        ro.append((t // bs) * shape.slot_bytes + (t % bs) * row)  # both chunks' records
        ri.append(np.full(tok_per_req, r % 3))
    sm, ro, ri = (np.concatenate(x).astype(np.int64) for x in (sm, ro, ri))
    tabs = position.delta_tables([11, 4000, 29000], 128, 500000.0, device="cuda")
    ops.scatter_slots_rerotate(ops.LayerTable(a), sm, ro, recs, tabs, ri)
    # reference: the whole pages through the per-page kernel (no fan-out) and
    # the ragged tail through the token kernel
    sm_o, ro_o, ri_o = ops.slot_order(sm, ro, ri)
    pages, poffs, pri, rest = ops.whole_pages(sm_o, ro_o, bs, row, ri_o)
    assert pages.size == n_req * (2 * n_chunk_pages - 1) and rest.sum() > 0
    assert 2 * np.unique(poffs).size <= poffs.size  # shared records: the fan-out path
    ops.scatter_rerotate(ops.LayerTable(b), pages, poffs, recs, tabs, pri, shared_records=False)
    ops.scatter_slots_rerotate(ops.LayerTable(b), sm_o[rest], ro_o[rest], recs, tabs, ri_o[rest])
    torch.cuda.synchronize()
    for l in range(4):
        assert torch.equal(a[l].view(torch.uint8), b[l].view(torch.uint8)), f"layer {l}"


def test_prepared_fanout_graph_capture_and_replay():
    """A prepared fan-out load (device tables) launches nothing but the
    kernel, so it can be captured into a HIP graph; each of three replays,
    with new records written eagerly in between, equals the eager call."""
    print("case: fanout graph capture", flush=True)
    shape, nb, recs, a, b, page_ids, offs, ridx, tabs, lg, ks, n_tables = _case(
        4, 128, "bf16", 0, 128, False, n_src=5, n=30, seed=31)
    prep = ops.PreparedFanout(ops.LayerTable(a), page_ids, offs, recs,
                              rope=(ridx, tabs, None, "neox", None, None))
    eager = ops.PreparedFanout(ops.LayerTable(b), page_ids, offs, recs,
                               rope=(ridx, tabs, None, "neox", None, None))
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        prep()  # warm-up on the capture stream
    torch.cuda.current_stream().wait_stream(side)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        prep()
    for rep in range(3):
        recs.view(torch.bfloat16).normal_(generator=torch.Generator(device="cuda")
                                          .manual_seed(40 + rep))
        g.replay()
        eager()
        torch.cuda.synchronize()
        for l in range(4):
            assert torch.equal(a[l].view(torch.uint8), b[l].view(torch.uint8)), (rep, l)


def _fanout_cases(n, seed):
    rng = np.random.default_rng(seed)
    out = []
    while len(out) < n:
        dt = ["bf16", "fp16", "e4m3", "e5m2"][rng.integers(4)]
        D = int(rng.choice([64, 96, 128, 256]))
        H = int(rng.choice([1, 2, 4, 8]))
        bs = int(rng.choice([1, 4, 8, 16, 32]))
        style = "gptj" if rng.random() < 0.3 else "neox"
        R = D if rng.random() < 0.7 else D // 2
        lay = ops.PagedKVLayout(num_layers=3, num_blocks=1, block_size=bs, num_heads=H,
                                head_dim=D, dtype=TORCH_DT[dt],
                                elem_bytes=1 if dt in ("e4m3", "e5m2") else 2,
                                kv_stride=0, page_stride=0, layer_bytes=0,
                                page_bytes=bs * H * D * (1 if dt in ("e4m3", "e5m2") else 2),
                                device=torch.device("cuda"))
        if lay.page_bytes % 16 or not ops.fanout_supported(lay, R, style):
            continue
        out.append((dt, D, H, bs, style, R, int(rng.integers(1 << 30))))
    return out


@pytest.mark.parametrize("case", _fanout_cases(16, 77))
def test_fanout_random_geometries_match_per_page(case):
    """Random geometries the fan-out takes (dtype, head_dim, heads, block
    size, style, partial rotary), through ops with host tables: the fan-out
    (shared-records hint) and the per-page kernels (no hint) give the same
    bits."""
    dt, D, H, bs, style, R, seed = case
    print(f"case: fanout random {case}", flush=True)
    e = 1 if dt in ("e4m3", "e5m2") else 2
    shape = KVShape(3, H, D, bs, e)
    rng = np.random.default_rng(seed)
    n_src, n = int(rng.integers(1, 6)), int(rng.integers(6, 40))
    nb = n + 3
    recs = torch.from_numpy(rng.standard_normal(n_src * shape.slot_bytes // 2)
                            .astype(np.float32)).to(torch.bfloat16).view(torch.uint8)
    if e == 1:  # finite 8-bit codes
        recs[(recs & 0x7F) == 0x7F] = 0x12
        recs[(recs & 0x7C) == 0x7C] = 0x22
    elif dt == "fp16":
        w = recs.view(torch.int16)
        w[((w >> 10) & 0x1F) == 0x1F] = 0x3C00
    recs = recs.cuda()
    page_ids = rng.permutation(nb)[:n].astype(np.int32)
    offs = rng.integers(0, n_src, n).astype(np.int64) * shape.slot_bytes
    ridx = rng.integers(-1, 3, n).astype(np.int32)
    tabs = position.delta_tables([17, 2048, 31111], R, 500000.0, device="cuda")
    ks = torch.tensor([0.02, 0.04, 0.01], device="cuda") if e == 1 else None
    a = rand_caches(shape, nb, dt, "cuda", seed=seed % 1000)
    b = [c.clone() for c in a]
    for caches, hint in ((a, True), (b, False)):
        ops.scatter_rerotate(ops.LayerTable(caches), page_ids, offs, recs, tabs, ridx,
                             rot_dim=R, style=style, k_scale=ks, shared_records=hint)
    torch.cuda.synchronize()
    for l in range(3):
        assert torch.equal(a[l].view(torch.uint8), b[l].view(torch.uint8)), f"layer {l}"


def _hnd_like(caches):
    """(2, NB, bs, H, D) views of head-major memory holding the same values."""
    out = []
    for c in caches:
        two, nb, bs, h, d = c.shape
        m = torch.empty((two, nb, h, bs, d), dtype=c.dtype, device=c.device)
        v = m.permute(0, 1, 3, 2, 4)
        v.copy_(c)
        out.append(v)
    return out


@pytest.mark.parametrize("layout", ["kx", "hnd"])
@pytest.mark.parametrize("dt,heads,head_dim,style,rot", [
    ("bf16", 8, 128, "neox", 128), ("e4m3", 8, 128, "neox", 128), ("bf16", 2, 64, "gptj", 64),
    ("fp16", 4, 128, "neox", 64), ("bf16", 1, 128, "neox", 128)])
def test_fanout_other_cache_layouts_match_per_page(layout, dt, heads, head_dim, style, rot):
    """Split-x (3-D PagedAttention caches) and head-major pages: the fan-out
    (shared-records hint) gives the bits of the per-page _kx / _hnd entry
    points (no hint), re-rotating and plain."""
    print(f"case: fanout {layout} {dt} H{heads} D{head_dim} {style} R{rot}", flush=True)
    e = 1 if dt in ("e4m3", "e5m2") else 2
    shape = KVShape(3, heads, head_dim, 16, e)
    rng = np.random.default_rng(heads * 31 + head_dim)
    n_src, n = 3, 24
    nb = n + 4
    recs = torch.from_numpy(rng.standard_normal(n_src * shape.slot_bytes // 2)
                            .astype(np.float32)).to(torch.bfloat16).view(torch.uint8)
    if e == 1:
        recs[(recs & 0x7F) == 0x7F] = 0x13
    elif dt == "fp16":
        w = recs.view(torch.int16)
        w[((w >> 10) & 0x1F) == 0x1F] = 0x3C00
    recs = recs.cuda()
    page_ids = rng.permutation(nb)[:n].astype(np.int32)
    offs = rng.integers(0, n_src, n).astype(np.int64) * shape.slot_bytes
    ridx = rng.integers(-1, 2, n).astype(np.int32)
    tabs = position.delta_tables([300, 17000], rot, 500000.0, device="cuda")
    ks = torch.tensor([0.02, 0.04, 0.01], device="cuda") if e == 1 else None
    base = rand_caches(shape, nb, dt, "cuda", seed=8)

    def table(caches):
        if layout == "kx":
            return ops.LayerTable([c.reshape(2, nb, -1) for c in caches], block_size=16,
                                  head_dim=head_dim)
        return ops.LayerTable(caches)

    outs = []
    for hint in (True, False):
        for rotate in (True, False):
            caches = [c.clone() for c in base]
            if layout == "hnd":
                caches = _hnd_like(caches)
            t = table(caches)
            if layout == "hnd" and heads > 1:
                assert t.layout.k_layout == "hnd"
            if rotate:
                ops.scatter_rerotate(t, page_ids, offs, recs, tabs, ridx, rot_dim=rot,
                                     style=style, k_scale=ks, shared_records=hint)
            else:
                ops.scatter(t, page_ids, offs, recs, shared_records=hint)
            outs.append([c.contiguous().view(torch.uint8) for c in caches])
    torch.cuda.synchronize()
    lay = table(base).layout
    assert ops.fanout_supported(lay, rot, style)
    for l in range(3):
        assert torch.equal(outs[0][l], outs[2][l]), f"rotated, layer {l}"
        assert torch.equal(outs[1][l], outs[3][l]), f"plain, layer {l}"
