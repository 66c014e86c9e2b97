"""Benchmark of the MI355X KV data-movement path.

A step is one offload gather plus one load scatter over the Llama-3-8B
workload (config 2: 32 layers, 8 KV heads, head_dim 128, block_size 16,
bf16, 64 requests with U[512, 8192] tokens on a randomly permuted block
pool, records packed into 256-token chunk buffers). Each pass is one kernel
launch covering every page of every request over all 32 layers.

value = algorithmic bytes of the step (gather reads P, writes P; scatter the
same: 4P) / step time, inputs resident in HBM. The fused re-rotate+scatter of
configs 3 (RAG reuse), 4 (e4m3), 5 (70B share) and 6 (one TP8 rank of 70B:
one KV head, 4 KiB pages) are reported beside it.

Per-kernel durations come from HIP events recorded on the launch stream
around every timed launch. cpu_baseline times the reference's own copy loops
(per page and layer torch copy_, daser_connector.py:536-551, 625-632),
restated on host tensors with torch on every host core of the process's
affinity, on a bounded sample of the same shape; cpu_port is the C oracle on
one thread, cpu_rerotate an fp32 torch rotate-half on all cores.

Re-rotations are also timed on the same memory viewed as vLLM's 3-D
PagedAttention caches (split-x K pages). --io adds the PCIe- and
file-inclusive save/load of the connector's data plane, --serving the host
cost of the connector's worker hooks on serving-shaped steps; neither is
`value`.

roofline prices the slower kernel of the step against the published 8 TB/s;
hbm_ceilings measures plain read-only, write-only and copy streams on the
same GPU in the same run, and roofline.frac_of_copy_bound prices the kernel
against the harmonic mean of the read and write rates, the most a copy can
sustain there.

Usage: python bench.py [--steps K] [--warmup W] [--configs 2,3,4,5,6] [--no-cpu]
                       [--no-ref-loop] [--io] [--serving] [--patterns] [--shapes]
                       [--calibrate] [--ceilings | --no-ceilings] [--reuse] [--tune k=v,...]
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "KV gather/scatter GB/s + % HBM peak; fused re-rotate+load tokens/s"
HBM_PEAK_GBS = 8000.0
THETA = 500000.0


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def fill_caches(torch, shape, num_blocks, dtype, dev, seed):
    """One (L, 2, NB, bs, H, D) allocation, viewed per layer, ~N(0,1).

    dtype "bf16", or "fp8": e4m3fn codes of N(0,1) values quantised with a
    per-layer scale amax / 448 (returned as the third element)."""
    g = torch.Generator(device=dev).manual_seed(seed)
    dims = (shape.num_layers, 2, num_blocks, shape.block_size, shape.num_heads,
            shape.head_dim)
    if dtype == "bf16":
        full = torch.empty(dims, dtype=torch.bfloat16, device=dev)
        flat = full.view(-1)
        for i in range(0, flat.numel(), 1 << 30):
            flat[i:i + (1 << 30)].normal_(generator=g)
        return full, [full[l] for l in range(shape.num_layers)], None
    full = torch.empty(dims, dtype=torch.float8_e4m3fn, device=dev)
    scales = torch.empty(shape.num_layers, dtype=torch.float32, device=dev)
    for l in range(shape.num_layers):
        tmp = torch.empty(dims[1:], dtype=torch.bfloat16, device=dev).normal_(generator=g)
        s = tmp.abs().amax().float() / 448.0
        full[l].copy_((tmp.float() / s).to(torch.float8_e4m3fn))
        scales[l] = s
        del tmp
    return full, [full[l] for l in range(shape.num_layers)], scales


class Timer:
    """HIP events around each launch on the current (launch) stream."""

    def __init__(self, torch):
        self.torch = torch
        self.pairs = []

    def __enter__(self):
        s = self.torch.cuda.Event(enable_timing=True)
        s.record()
        self.pairs.append([s, None])
        return self

    def __exit__(self, *exc):
        e = self.torch.cuda.Event(enable_timing=True)
        e.record()
        self.pairs[-1][1] = e

    def mean_ms(self):
        ts = [s.elapsed_time(e) for s, e in self.pairs]
        return float(np.mean(ts)) if ts else float("nan")

    def reset(self):
        self.pairs = []


def bench_copy(torch, ops, wl, dtype, dev, steps, warmup, position=None):
    """Config 2/4: gather then scatter per step. Returns the result dict.
    For fp8 (config 4) the re-rotating scatter of the same pages is timed
    too: each request moves by a random delta in [0, 32768)."""
    shape = wl.shape
    log(f"[bench] allocating caches {wl.num_blocks} blocks x {shape.num_layers} layers "
        f"({wl.num_blocks * shape.slot_bytes / 1e9:.1f} GB) + staging "
        f"{wl.staging_bytes / 1e9:.1f} GB")
    full, caches, k_scale = fill_caches(torch, shape, wl.num_blocks, dtype, dev, seed=1)
    table = ops.LayerTable(caches)
    staging = torch.empty(wl.staging_bytes, dtype=torch.uint8, device=dev)
    ids = torch.from_numpy(wl.page_ids).to(dev)
    offs = torch.from_numpy(wl.slot_offsets).to(dev)
    # the scatter's page list in destination-block order (as ops.scatter
    # orders host tables)
    s_ids_np, s_offs_np, _ = ops.dest_order(wl.page_ids, wl.slot_offsets)
    s_ids = torch.from_numpy(s_ids_np.astype(np.int32)).to(dev)
    s_offs = torch.from_numpy(s_offs_np).to(dev)
    tg, ts = Timer(torch), Timer(torch)
    for i in range(warmup):
        ops.gather(table, ids, offs, staging)
        ops.scatter(table, s_ids, s_offs, staging)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(steps):
        with tg:
            ops.gather(table, ids, offs, staging)
        with ts:
            ops.scatter(table, s_ids, s_offs, staging)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    # a cheap end-to-end check: the scatter wrote back what the gather read
    probe = int(wl.page_ids[len(wl.page_ids) // 2])
    p_idx = len(wl.page_ids) // 2
    rec = staging[int(wl.slot_offsets[p_idx]):int(wl.slot_offsets[p_idx]) + shape.layer_bytes]
    ok = torch.equal(rec, caches[0][:, probe].reshape(-1).view(torch.uint8))
    P = wl.payload_bytes
    g_ms, s_ms = tg.mean_ms(), ts.mean_ms()
    rot = {}
    if dtype == "bf16":
        # the same requests through vLLM's slot_mapping (token-granular form):
        # moves only the valid tokens' rows
        tables, k = [], 0
        for n in wl.req_pages:
            tables.append(wl.page_ids[k:k + n].tolist())
            k += n
        row = shape.num_heads * shape.head_dim * shape.elem_bytes
        sm_np = ops.slot_mapping_for(tables, wl.req_tokens, shape.block_size)
        ro_np = ops.token_row_offsets(wl.req_tokens, shape.slot_bytes, shape.block_size, row)
        sm = torch.from_numpy(sm_np).to(dev)
        ro = torch.from_numpy(ro_np).to(dev)
        # the token-form load as ops.scatter_slots runs host tables: in
        # destination-slot order, whole pages through the page scatter and
        # the ragged rows through the token kernel; the split is made once,
        # as by a caller whose tables stay resident
        from daser_amd import position as _position

        rng = np.random.default_rng(11)
        deltas = rng.integers(1, 32768, size=len(wl.req_tokens)).tolist()
        req_idx, uniq = _position.page_rope_index([1] * len(deltas), deltas)
        tabs = _position.delta_tables(uniq, shape.head_dim, THETA, device=dev)
        tok_idx = np.repeat(np.asarray(req_idx, np.int64), wl.req_tokens)
        sm_o, ro_o, ri_o = ops.slot_order(sm_np, ro_np, tok_idx)
        pg, pg_offs, pg_ri, rest = ops.whole_pages(sm_o, ro_o, shape.block_size, row, ri_o)

        def dev_t(x, dt=torch.int64):
            return torch.from_numpy(np.ascontiguousarray(x)).to(dt).to(dev)

        pg_d, pg_offs_d, pg_ri_d = dev_t(pg, torch.int32), dev_t(pg_offs), dev_t(pg_ri, torch.int32)
        sm_r, ro_r, ri_r = dev_t(sm_o[rest]), dev_t(ro_o[rest]), dev_t(ri_o[rest], torch.int32)
        has_rest = bool(np.any(sm_o[rest] >= 0))

        def scatter_tokens():
            ops.scatter(table, pg_d, pg_offs_d, staging)
            if has_rest:
                ops.scatter_slots(table, sm_r, ro_r, staging)

        def rerotate_tokens():
            ops.scatter_rerotate(table, pg_d, pg_offs_d, staging, tabs, pg_ri_d)
            if has_rest:
                ops.scatter_slots_rerotate(table, sm_r, ro_r, staging, tabs, ri_r)

        tsg, tss = Timer(torch), Timer(torch)
        for i in range(warmup + steps):
            if i < warmup:
                ops.gather_slots(table, sm, ro, staging)
                scatter_tokens()
                continue
            with tsg:
                ops.gather_slots(table, sm, ro, staging)
            with tss:
                scatter_tokens()
        tsr = Timer(torch)
        for i in range(warmup + steps):
            if i < warmup:
                rerotate_tokens()
                continue
            with tsr:
                rerotate_tokens()
        torch.cuda.synchronize()
        tokP = wl.tokens * row * 2 * shape.num_layers
        rot = {"slots_gather_ms": tsg.mean_ms(), "slots_scatter_ms": tss.mean_ms(),
               "slots_rerotate_ms": tsr.mean_ms(),
               "slots_payload_bytes": tokP,
               "slots_whole_pages": int(pg.size), "slots_ragged_tokens": int(np.sum(sm_o[rest] >= 0)),
               "slots_gather_GBps": 2 * tokP / (tsg.mean_ms() * 1e-3) / 1e9,
               "slots_scatter_GBps": 2 * tokP / (tss.mean_ms() * 1e-3) / 1e9,
               "slots_rerotate_GBps": 2 * tokP / (tsr.mean_ms() * 1e-3) / 1e9}
    if dtype == "fp8" and position is not None:
        rng = np.random.default_rng(7)
        deltas = rng.integers(1, 32768, size=len(wl.req_pages)).tolist()
        ridx, uniq = position.page_rope_index(wl.req_pages, deltas)
        tabs = position.delta_tables(uniq, shape.head_dim, THETA, device=dev)
        _, _, s_ridx = ops.dest_order(wl.page_ids, wl.slot_offsets, ridx)
        ridx_d = torch.from_numpy(s_ridx.astype(np.int32)).to(dev)
        tr = Timer(torch)
        for i in range(warmup + steps):
            if i < warmup:
                ops.scatter_rerotate(table, s_ids, s_offs, staging, tabs, ridx_d, k_scale=k_scale)
                continue
            with tr:
                ops.scatter_rerotate(table, s_ids, s_offs, staging, tabs, ridx_d, k_scale=k_scale)
        torch.cuda.synchronize()
        r_ms = tr.mean_ms()
        # the same bytes as an e5m2 cache (vLLM's fp8_e5m2): same kernels,
        # the other 8-bit codec
        t5 = ops.LayerTable([c.view(torch.float8_e5m2) for c in caches])
        te = Timer(torch)
        for i in range(warmup + steps):
            if i < warmup:
                ops.scatter_rerotate(t5, s_ids, s_offs, staging, tabs, ridx_d, k_scale=k_scale)
                continue
            with te:
                ops.scatter_rerotate(t5, s_ids, s_offs, staging, tabs, ridx_d, k_scale=k_scale)
        torch.cuda.synchronize()
        e5_ms = te.mean_ms()
        del t5
        rot = {"rerotate_ms": r_ms, "rerotate_GBps": 2 * P / (r_ms * 1e-3) / 1e9,
               "rerotate_tokens_per_s": wl.tokens / (r_ms * 1e-3),
               "rerotate_e5m2_ms": e5_ms,
               "rerotate_e5m2_GBps": 2 * P / (e5_ms * 1e-3) / 1e9}
    del full, caches, table, staging
    torch.cuda.empty_cache()
    return {
        "payload_bytes": P,
        "pages": wl.n_pages,
        "tokens": wl.tokens,
        "step_ms": wall * 1e3 / steps,
        "gather_ms": g_ms,
        "scatter_ms": s_ms,
        "gather_GBps": 2 * P / (g_ms * 1e-3) / 1e9,
        "scatter_GBps": 2 * P / (s_ms * 1e-3) / 1e9,
        "step_GBps": 4 * P / wall * steps / 1e9,
        "probe_ok": bool(ok),
        **rot,
    }


def bench_rerotate(torch, ops, position, wl, dtype, dev, steps, warmup):
    """Config 3/5: fused re-rotate+scatter of reused chunks."""
    shape = wl.shape
    src_bytes = wl.meta["src_staging_bytes"]
    log(f"[bench] rerotate: source records {src_bytes / 1e9:.1f} GB, destination "
        f"{wl.num_blocks * shape.slot_bytes / 1e9:.1f} GB")
    full, caches, k_scale = fill_caches(torch, shape, wl.num_blocks, dtype, dev, seed=2)
    table = ops.LayerTable(caches)
    src = torch.empty(src_bytes, dtype=torch.uint8, device=dev)
    g = torch.Generator(device=dev).manual_seed(3)
    for i in range(0, src_bytes, 1 << 30):
        n = min(1 << 30, src_bytes - i)
        if dtype == "fp8":
            src[i:i + n].random_(0, 256, generator=g)
            src[i:i + n][src[i:i + n] == 0x7F] = 0  # no NaN codes in the synthetic data
        else:
            src[i:i + n].view(torch.bfloat16).normal_(generator=g)
    ridx, uniq = position.page_rope_index(wl.chunk_pages, wl.chunk_delta)
    tabs = position.delta_tables(uniq, shape.head_dim, THETA, device=dev)
    s_ids, s_offs, s_ridx = ops.dest_order(wl.page_ids, wl.src_offsets, ridx)
    ids = torch.from_numpy(s_ids.astype(np.int32)).to(dev)
    offs = torch.from_numpy(s_offs).to(dev)
    ridx_d = torch.from_numpy(s_ridx.astype(np.int32)).to(dev)
    # the launch hint ops.scatter_rerotate infers from host offsets: configs
    # 5 and 6 place 64 cached chunks in every request (records read by
    # several pages), config 3's chunks are all distinct
    shared = bool(2 * np.unique(wl.src_offsets).size <= wl.src_offsets.size)
    t = Timer(torch)
    for _ in range(warmup):
        ops.scatter_rerotate(table, ids, offs, src, tabs, ridx_d, k_scale=k_scale,
                             shared_records=shared)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        with t:
            ops.scatter_rerotate(table, ids, offs, src, tabs, ridx_d, k_scale=k_scale,
                                 shared_records=shared)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms = t.mean_ms()
    fan = {}
    if shared and ops.fanout_supported(table.layout, shape.head_dim):
        # what ops.scatter_rerotate runs for host tables with shared records:
        # each distinct record read once and written to all of its pages
        # (dsr_scatter_fanout), tables grouped and uploaded once
        prep = ops.PreparedFanout(table, s_ids, s_offs, src,
                                  rope=(s_ridx, tabs, None, "neox", k_scale, None))
        tf = Timer(torch)
        for _ in range(warmup):
            prep()
        for _ in range(steps):
            with tf:
                prep()
        plain = ops.PreparedFanout(table, s_ids, s_offs, src)
        tp = Timer(torch)
        for _ in range(warmup):
            plain()
        for _ in range(steps):
            with tp:
                plain()
        torch.cuda.synchronize()
        fan = {"fanout_ms": tf.mean_ms(), "fanout_plain_ms": tp.mean_ms(),
               "fanout_sources": prep.n_src,
               "fanout_read_bytes": prep.n_src * shape.slot_bytes}
    # the same page list as a plain scatter: the copy ceiling of this layout
    tc = Timer(torch)
    for _ in range(steps):
        with tc:
            ops.scatter(table, ids, offs, src, shared_records=shared)
    torch.cuda.synchronize()
    copy_ms = tc.mean_ms()
    P = wl.n_pages * shape.slot_bytes
    # the same pages as 3-D caches with split-x K pages (vLLM's PagedAttention
    # layout): same memory, the kx re-rotation entry point
    flat = ops.LayerTable([c.reshape(2, c.shape[1], -1) for c in caches],
                          block_size=shape.block_size, head_dim=shape.head_dim)
    tk = Timer(torch)
    for _ in range(warmup):
        ops.scatter_rerotate(flat, ids, offs, src, tabs, ridx_d, k_scale=k_scale,
                             shared_records=shared)
    for _ in range(steps):
        with tk:
            ops.scatter_rerotate(flat, ids, offs, src, tabs, ridx_d, k_scale=k_scale,
                                 shared_records=shared)
    torch.cuda.synchronize()
    extra = {"kx_kernel_ms": tk.mean_ms(), "kx_GBps": 2 * P / (tk.mean_ms() * 1e-3) / 1e9,
             "shared_records": shared}
    del flat
    if P < torch.cuda.mem_get_info(dev)[0] // 2:
        # the save direction over the same pages into one record per page
        del src
        recs = torch.empty(P, dtype=torch.uint8, device=dev)
        roffs = torch.arange(wl.n_pages, dtype=torch.int64, device=dev) * shape.slot_bytes
        tg = Timer(torch)
        for _ in range(warmup):
            ops.gather(table, ids, roffs, recs)
        for _ in range(steps):
            with tg:
                ops.gather(table, ids, roffs, recs)
        torch.cuda.synchronize()
        extra.update({"gather_ms": tg.mean_ms(),
                      "gather_GBps": 2 * P / (tg.mean_ms() * 1e-3) / 1e9})
        if shape.num_heads * shape.head_dim * shape.elem_bytes <= 512:
            # small rows: the token-form kernels over the same pages, all
            # tokens valid (slot = block * bs + t, record row t)
            bs = shape.block_size
            row = shape.num_heads * shape.head_dim * shape.elem_bytes
            t = torch.arange(wl.n_pages * bs, device=dev)
            sm = ids.to(torch.int64).repeat_interleave(bs) * bs + t % bs
            ro = roffs.repeat_interleave(bs) + (t % bs) * row
            tsg, tss = Timer(torch), Timer(torch)
            for _ in range(warmup):
                ops.gather_slots(table, sm, ro, recs)
            for _ in range(steps):
                with tsg:
                    ops.gather_slots(table, sm, ro, recs)
            for _ in range(steps):
                with tss:
                    ops.scatter_slots(table, sm, ro, recs)
            torch.cuda.synchronize()
            extra.update({"slots_gather_GBps": 2 * P / (tsg.mean_ms() * 1e-3) / 1e9,
                          "slots_scatter_GBps": 2 * P / (tss.mean_ms() * 1e-3) / 1e9})
        src = recs
    del full, caches, table, src
    torch.cuda.empty_cache()
    return {**extra, **fan,
        "payload_bytes": P,
        "pages": wl.n_pages,
        "tokens": wl.tokens,
        "kernel_ms": ms,
        "wall_ms_per_launch": wall * 1e3 / steps,
        "tokens_per_s": wl.tokens / (ms * 1e-3),
        "GBps": 2 * P / (ms * 1e-3) / 1e9,
        "frac_hbm_peak": 2 * P / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS,
        "plain_scatter_ms": copy_ms,
        "plain_scatter_GBps": 2 * P / (copy_ms * 1e-3) / 1e9,
    }


def store_fs(path: str) -> str:
    """File system type and device of the mount holding ``path``
    (/proc/mounts, longest matching mount point)."""
    best, out = "", "unknown"
    try:
        for line in open("/proc/mounts"):
            dev, mnt, fstype = line.split()[:3]
            if (path == mnt or path.startswith(mnt.rstrip("/") + "/")) and len(mnt) > len(best):
                best, out = mnt, f"{fstype} on {dev} (mounted at {mnt})"
    except OSError:
        pass
    return out


def bench_io(torch, dev, budget_bytes: int = 2 << 30, reps: int = 3,
             backends=("native", "mmap", "direct")) -> dict:
    """PCIe- and file-inclusive rates of the connector's data plane on a
    sample of config 2's shape: save = gather + device->pinned ring->file,
    load = file->pinned ring->device + scatter, through KVDataPlane with
    each ring backend (default ring geometry: 8 x 4 MiB slots), into a store
    file under $TMPDIR. Not the headline value."""
    import shutil
    import tempfile

    from daser_amd import workloads
    from daser_amd.connector import KVDataPlane, ReqLoadSpec, ReqStoreSpec, plan_load, plan_store

    shape = workloads.LLAMA3_8B
    n_pages = max(1, budget_bytes // shape.slot_bytes)
    nb = n_pages + 64
    full, caches, _ = fill_caches(torch, shape, nb, "bf16", dev, seed=9)
    named = {f"layer.{i}": c for i, c in enumerate(caches)}
    rng = np.random.default_rng(3)
    blocks = rng.permutation(nb)[:n_pages].tolist()
    per = 16  # 256-token chunks, one transfer each
    store = {f"r{i}": ReqStoreSpec(f"k{i}", i, min(per, n_pages - i), blocks[i:i + per],
                                   i * shape.slot_bytes, per * 16)
             for i in range(0, n_pages, per)}
    sp = plan_store(store, shape.slot_bytes)
    load = {k: ReqLoadSpec(v.chunk_key, v.start_slot, v.num_slots, v.block_ids,
                           v.file_offset, v.token_count) for k, v in store.items()}
    lp = plan_load(load, shape.slot_bytes)
    P = n_pages * shape.slot_bytes
    out = {"payload_bytes": P, "backends": {},
           "store_fs": store_fs(os.path.realpath(tempfile.gettempdir())),
           "sample": f"{n_pages} Llama-3-8B pages ({P / 1e9:.2f} GB) in 256-token chunks "
                     f"(one {per * shape.slot_bytes >> 20} MiB transfer each), best of {reps}, "
                     f"store file under {tempfile.gettempdir()}"}
    for backend in backends:
        d = tempfile.mkdtemp(prefix="daser_bench_")
        try:
            plane = KVDataPlane(os.path.join(d, "daser.store"), io_backend=backend)
            plane.register(named)
            arena = plane.new_store_arena(sp)
            ts, tl = [], []
            for _ in range(reps):
                torch.cuda.synchronize()
                t0 = time.perf_counter()
                plane.save_all(sp, arena)
                plane.flush(sp, arena)
                torch.cuda.synchronize()
                ts.append(time.perf_counter() - t0)
                t0 = time.perf_counter()
                plane.load(lp)
                torch.cuda.synchronize()
                tl.append(time.perf_counter() - t0)
            out["backends"][backend] = {"save_GBps": round(P / min(ts) / 1e9, 2),
                                        "load_GBps": round(P / min(tl) / 1e9, 2),
                                        "ring": plane.io.backend}
            plane.close()
            del arena
        except Exception as e:  # a backend the file system refuses (O_DIRECT)
            out["backends"][backend] = {"error": f"{type(e).__name__}: {e}"}
        finally:
            shutil.rmtree(d, ignore_errors=True)
    del full, caches
    torch.cuda.empty_cache()
    dflt = out["backends"].get("mmap", {})  # the connector's default backend
    out["save_GBps"], out["load_GBps"] = dflt.get("save_GBps"), dflt.get("load_GBps")
    out["default_backend"] = "mmap"
    return out


class _BenchIPC:
    """Stands in for the store server's async client: commits succeed."""

    async def commit_chunk(self, key):
        return {"ok": True}


class _IndexServer:
    """Stands in for the store server's sync client: match_and_alloc over a
    retrieval index, with the reply the reference server builds
    (daser/server/ipc_server.py:256-291); hits allocate nothing."""

    def __init__(self, index, slot_bytes):
        self.index, self.slot = index, slot_bytes

    def match_and_alloc(self, tokens, chunk_key, model_id):
        import asyncio

        hits = asyncio.run(self.index.lookup(tokens, model_id))
        return {"chunks": [{"chunk_key": m.chunk_key, "start_slot": m.start_slot,
                            "num_slots": m.num_slots, "token_count": m.token_count,
                            "pos_offset": m.pos_offset, "model_id": m.model_id,
                            "file_offset": m.start_slot * self.slot} for m in hits],
                "alloc": None}


def bench_serving(torch, dev, steps: int = 10, n_req: int = 8, chunk_pages: int = 16,
                  hit_pages: int = 128) -> dict:
    """Host cost and latency of the connector's worker hooks on serving-shaped
    steps at config 2's shape (Llama-3-8B bf16), through DaserConnector with
    the native ring and a store file under $TMPDIR:
    save step = bind metadata, save_kv_layer for each of the 32 layers, then
    wait_for_save, for n_req requests storing one 256-token chunk each
    (blocking and async_save);
    load step = start_load_kv of n_req requests hitting hit_pages pages each,
    placed at a new position (fused re-rotation), until the device is done.
    Beside it, the reference's per-(page, layer) copy loops for the same
    pages (daser_connector.py:625-632 and :536-551) on the same GPU."""
    import shutil
    import tempfile
    from types import SimpleNamespace

    from daser_amd import connector as C
    from daser_amd import workloads
    from daser_amd.store_io import preallocate_store

    shape = workloads.LLAMA3_8B
    nb = n_req * hit_pages + 64
    full, caches, _ = fill_caches(torch, shape, nb, "bf16", dev, seed=11)
    named = {f"model.layers.{i}.self_attn.attn": c for i, c in enumerate(caches)}
    rng = np.random.default_rng(5)
    d = tempfile.mkdtemp(prefix="daser_serving_")
    store = os.path.join(d, "daser.store")
    slot = shape.slot_bytes
    preallocate_store(store, n_req * hit_pages * slot)
    with open(store, "r+b") as f:  # loads read written records, not file holes
        piece = np.random.default_rng(6).integers(0, 256, 1 << 24, dtype=np.uint8).tobytes()
        for _ in range(n_req * hit_pages * slot // len(piece)):
            f.write(piece)
    out = {}

    def worker(**extra):
        cfg = SimpleNamespace(kv_transfer_config=SimpleNamespace(kv_connector_extra_config=dict(
            store_path=store, rope_theta=500000.0, **extra)))
        w = C.DaserConnector(cfg, C.KVConnectorRole.WORKER, ipc_async=_BenchIPC())
        w.register_kv_caches(named)
        return w

    def store_meta():
        blocks = rng.permutation(nb)[:n_req * chunk_pages].tolist()
        reqs = {}
        for r in range(n_req):
            s0 = r * chunk_pages
            reqs[f"s{r}"] = C.ReqStoreSpec(f"k{r}", s0, chunk_pages,
                                           blocks[s0:s0 + chunk_pages], s0 * slot,
                                           chunk_pages * 16)
        return C.DaserConnectorMeta(reqs_to_store=reqs)

    def rag_case(w, n_docs: int = 16, per_prompt: int = 10, n_prompts: int = 4):
        """RAG prompts through both connector roles: n_docs cached 512-token
        chunks (records already in the store file, stored at position 0) in a
        ChunkAssemblyIndex; each prompt = per_prompt chunks drawn at random
        + a 20-token question. The scheduler places the chunks (segments at
        0, 512, ...) and the worker loads them, re-rotating each chunk's K
        from 0 to its place. Times the scheduler hooks per request and the
        worker's start_load_kv per step (n_prompts requests)."""
        import asyncio

        from daser_amd.retrieval import ChunkAssemblyIndex, ChunkMeta, chunk_key

        bs, ct = shape.block_size, 512
        idx = ChunkAssemblyIndex(bs)
        trng = np.random.default_rng(9)
        docs = [trng.integers(0, 120000, ct).tolist() for _ in range(n_docs)]
        for i, t in enumerate(docs):
            asyncio.run(idx.insert(ChunkMeta(chunk_key(t), i * (ct // bs), ct // bs, ct, 0,
                                             "default")))
        cfg = SimpleNamespace(kv_transfer_config=SimpleNamespace(
            kv_connector_extra_config={"block_tokens": bs, "allow_chunk_assembly": True}))
        sched = C.DaserConnector(cfg, C.KVConnectorRole.SCHEDULER,
                                 ipc_client=_IndexServer(idx, slot))
        sched_ms, load_ms, placed = [], [], []
        need = per_prompt * ct // bs + 2
        n_prompts = min(n_prompts, nb // need)
        for it in range(steps + 1):
            blocks = rng.permutation(nb)
            meta_all = C.DaserConnectorMeta()
            t0 = time.perf_counter()
            for r in range(n_prompts):
                pick = trng.choice(n_docs, per_prompt, replace=False)
                prompt = [t for i in pick for t in docs[i]] + trng.integers(0, 120000, 20).tolist()
                req = SimpleNamespace(request_id=f"rag{it}_{r}", prompt_token_ids=prompt)
                n, _ = sched.get_num_new_matched_tokens(req, 0)
                placed.append(n)
                mine = blocks[r * need:(r + 1) * need].tolist()
                sched.update_state_after_alloc(
                    req, SimpleNamespace(blocks=[[SimpleNamespace(block_id=b) for b in mine]]), n)
                m = sched.build_connector_meta(
                    SimpleNamespace(num_scheduled_tokens={req.request_id: len(prompt)}))
                meta_all.reqs_to_load.update(m.reqs_to_load)
            t1 = time.perf_counter()
            torch.cuda.synchronize()
            t2 = time.perf_counter()
            w.bind_connector_metadata(meta_all)
            w.start_load_kv(None)
            torch.cuda.synchronize()
            t3 = time.perf_counter()
            w.clear_connector_metadata()
            if it:
                sched_ms.append((t1 - t0) * 1e3 / n_prompts)
                load_ms.append((t3 - t2) * 1e3)
        tok = n_prompts * per_prompt * ct
        return {"tokens_placed_per_request": int(np.median(placed)),
                "scheduler_ms_per_request_median": round(float(np.median(sched_ms)), 3),
                "start_load_kv_ms_median": round(float(np.median(load_ms)), 3),
                "loaded_tokens_per_s": round(tok / (np.median(load_ms) * 1e-3)),
                "sample": f"{n_prompts} requests per step, each {per_prompt} of {n_docs} cached "
                          f"{ct}-token chunks + 20 question tokens; records from the page cache"}

    try:
        for mode in ("blocking", "async_save"):
            w = worker(async_save=mode == "async_save")
            hook_us, wait_ms, step_ms = [], [], []
            for it in range(steps + 1):
                meta = store_meta()
                torch.cuda.synchronize()
                t0 = time.perf_counter()
                w.bind_connector_metadata(meta)
                for name, t in named.items():
                    h0 = time.perf_counter()
                    w.save_kv_layer(name, t, None)
                    hook_us.append((time.perf_counter() - h0) * 1e6)
                h1 = time.perf_counter()
                w.wait_for_save()
                t1 = time.perf_counter()
                w.clear_connector_metadata()
                if it:  # the first step opens the rings
                    wait_ms.append((t1 - h1) * 1e3)
                    step_ms.append((t1 - t0) * 1e3)
                else:
                    hook_us.clear()
            w._plane.drain(timeout=120.0)
            w.shutdown()
            out[f"save_{mode}"] = {
                "save_kv_layer_host_us_median": round(float(np.median(hook_us)), 1),
                "wait_for_save_ms_median": round(float(np.median(wait_ms)), 3),
                "step_ms_median": round(float(np.median(step_ms)), 3),
                "bytes_per_step": n_req * chunk_pages * slot}

        w = worker()

        def load_case(n, pages, rotate):
            ms = []
            for it in range(steps + 1):
                blocks = rng.permutation(nb)[:n * pages].tolist()
                reqs = {}
                for r in range(n):
                    s0 = r * pages
                    reqs[f"l{r}"] = C.ReqLoadSpec(
                        f"k{r}", s0, pages, blocks[s0:s0 + pages], s0 * slot, pages * 16,
                        pos_offset=0, new_pos=int(rng.integers(1, 32768)) if rotate else None)
                torch.cuda.synchronize()
                t0 = time.perf_counter()
                w.bind_connector_metadata(C.DaserConnectorMeta(reqs_to_load=reqs))
                w.start_load_kv(None)
                torch.cuda.synchronize()
                if it:
                    ms.append((time.perf_counter() - t0) * 1e3)
                w.clear_connector_metadata()
            b = n * pages * slot
            return {"start_load_kv_ms_median": round(float(np.median(ms)), 3),
                    "GBps_file_inclusive": round(b / np.median(ms) / 1e6, 2),
                    "bytes_per_step": b}

        out["load_rerotate"] = load_case(n_req, hit_pages, True)
        out["load_one_chunk_rerotate"] = load_case(1, chunk_pages, True)
        out["load_one_chunk"] = load_case(1, chunk_pages, False)
        out["rag_assembly"] = rag_case(w)
        w.shutdown()

        # the reference's loops for the same step sizes (device copies only, no I/O)
        layer = shape.layer_bytes
        pages = rng.permutation(nb)[:n_req * chunk_pages].tolist()
        staging = torch.empty(len(pages) * slot, dtype=torch.uint8, device=dev)

        def ref_save():
            for l, t in enumerate(caches):  # one save_kv_layer per layer
                for i, b in enumerate(pages):
                    src = t[:, b]
                    o = i * slot + l * layer
                    staging[o:o + src.nbytes].copy_(src.reshape(-1).view(torch.uint8))

        ref_save()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(3):
            ref_save()
        torch.cuda.synchronize()
        out["reference_save_loop_ms"] = round((time.perf_counter() - t0) / 3 * 1e3, 3)
    finally:
        shutil.rmtree(d, ignore_errors=True)
        del full, caches, named
        torch.cuda.empty_cache()
    out["sample"] = (f"{steps} steps each after one warm-up; save: {n_req} requests x "
                     f"{chunk_pages} pages (256 tokens); load: {n_req} requests x {hit_pages} "
                     f"pages re-rotated to new positions, and one 256-token chunk with and without a "
                     f"position change; store file under "
                     f"{tempfile.gettempdir()} (page cache)")
    return out


# Cache shapes of other model families (layers, KV heads, head_dim, block size,
# element bytes), for --shapes: page sizes from 4 to 96 KiB and head_dim 64
# to 256, each with its own kernel choices.
MODEL_SHAPES = [
    ("qwen2-0.5b", (24, 2, 64, 16, 2)),
    ("llama-3.2-1b", (16, 8, 64, 16, 2)),
    ("qwen2.5-7b", (28, 4, 128, 16, 2)),
    ("llama-3-8b", (32, 8, 128, 16, 2)),
    ("llama-3-8b bs32", (32, 8, 128, 32, 2)),
    ("gemma-2-9b", (42, 8, 256, 16, 2)),
    ("phi-3-mini", (32, 32, 96, 16, 2)),
    ("llama-3-70b tp8", (80, 1, 128, 16, 2)),
    ("llama-3-8b e4m3", (32, 8, 128, 16, 1)),
]


def bench_shapes(torch, ops, position, dev, payload: int = 16 << 30, steps: int = 3) -> dict:
    """Gather, scatter and the fused re-rotating scatter (every request moved
    by its own delta) at the cache shapes of other model families: ragged
    requests (U[256, 4096] tokens) on a permuted pool, about ``payload``
    bytes of records per pass. GB/s = 2P / mean HIP-event kernel time."""
    from daser_amd import workloads

    out = {}
    for name, dims in MODEL_SHAPES:
        shape = workloads.KVShape(*dims)
        tok_bytes = shape.slot_bytes // shape.block_size
        n_req = max(1, int(payload // tok_bytes // 2176))
        wl = workloads.ragged(shape, n_req, 256, 4096, seed=17, pool_slack=1.05)
        fp8 = shape.elem_bytes == 1
        full, caches, k_scale = fill_caches(torch, shape, wl.num_blocks,
                                            "fp8" if fp8 else "bf16", dev, seed=5)
        table = ops.LayerTable(caches)
        st = torch.empty(wl.staging_bytes, dtype=torch.uint8, device=dev)
        g_ids = torch.from_numpy(wl.page_ids.astype(np.int32)).to(dev)
        g_offs = torch.from_numpy(wl.slot_offsets).to(dev)
        rng = np.random.default_rng(3)
        ridx, uniq = position.page_rope_index(wl.req_pages,
                                              rng.integers(1, 32768, len(wl.req_pages)).tolist())
        tabs = position.delta_tables(uniq, shape.head_dim, THETA, device=dev)
        s_ids, s_offs, s_ridx = ops.dest_order(wl.page_ids, wl.slot_offsets, ridx)
        s_ids = torch.from_numpy(s_ids.astype(np.int32)).to(dev)
        s_offs = torch.from_numpy(s_offs).to(dev)
        s_ridx = torch.from_numpy(s_ridx.astype(np.int32)).to(dev)
        runs = {"gather": lambda: ops.gather(table, g_ids, g_offs, st),
                "scatter": lambda: ops.scatter(table, s_ids, s_offs, st),
                "rerotate": lambda: ops.scatter_rerotate(table, s_ids, s_offs, st, tabs, s_ridx,
                                                         k_scale=k_scale)}
        P = wl.n_pages * shape.slot_bytes
        res = {"page_KiB": shape.page_bytes // 1024, "pages": wl.n_pages,
               "payload_GB": round(P / 1e9, 2)}
        for k, fn in runs.items():
            fn()
            t = Timer(torch)
            for _ in range(steps):
                with t:
                    fn()
            torch.cuda.synchronize()
            res[f"{k}_GBps"] = round(2 * P / (t.mean_ms() * 1e-3) / 1e9, 1)
        res["rerotate_tokens_per_s"] = round(wl.tokens / (2 * P / (res["rerotate_GBps"] * 1e9)))
        out[name] = res
        log(f"[bench] shapes: {name}: {json.dumps(res)}")
        del full, caches, table, st
        torch.cuda.empty_cache()
    return out


def bench_patterns(torch, ops, dev, reps: int = 5) -> dict:
    """The same bytes as config 2 (P = 17,742 pages x 2 MiB records) moved in
    other patterns, for scale: torch's own kernels for a plain sequential
    copy (copy_), a sequential-read -> permuted-32 KiB-row write
    (index_copy_) and a permuted-read -> sequential write (index_select), and
    this library's scatter / gather over the same caches with an identity
    page list (both sides sequential; 8 pages fewer) and with config 2's
    permutation. Mean
    kernel time over `reps` launches (HIP events), GB/s = 2P / time."""
    from daser_amd import workloads

    wl = workloads.config(2)
    sh = wl.shape
    P = wl.payload_bytes
    rows = P // sh.page_bytes  # 32 KiB rows
    out = {"payload_bytes": P, "row_bytes": sh.page_bytes}

    def timed(fn):
        t = Timer(torch)
        fn()
        for _ in range(reps):
            with t:
                fn()
        torch.cuda.synchronize()
        return round(2 * P / (t.mean_ms() * 1e-3) / 1e9, 1)

    g = torch.Generator().manual_seed(0)
    src = torch.empty(P, dtype=torch.uint8, device=dev).fill_(3)
    pool_rows = int(rows * 1.05)
    dst = torch.empty(pool_rows * sh.page_bytes, dtype=torch.uint8, device=dev)
    perm = torch.randperm(pool_rows, generator=g)[:rows].to(dev)
    src2 = src.view(rows, sh.page_bytes)
    dst2 = dst.view(pool_rows, sh.page_bytes)
    out["torch_copy_sequential_GBps"] = timed(lambda: dst[:P].copy_(src))
    out["torch_index_copy_permuted_write_GBps"] = timed(lambda: dst2.index_copy_(0, perm, src2))
    out["torch_index_select_permuted_read_GBps"] = timed(
        lambda: torch.index_select(dst2, 0, perm, out=src2))
    del src, dst, src2, dst2
    torch.cuda.empty_cache()
    full, caches, _ = fill_caches(torch, sh, wl.num_blocks, "bf16", dev, seed=1)
    table = ops.LayerTable(caches)
    st = torch.empty(wl.staging_bytes, dtype=torch.uint8, device=dev)
    offs = torch.from_numpy(wl.slot_offsets).to(dev)
    # the identity list covers 8 pages fewer, so that a profile tells its
    # launches (grid) from config 2's; its rate is scaled to its own bytes
    n_id = wl.n_pages - 8
    ident = torch.arange(n_id, dtype=torch.int32, device=dev)
    ids = torch.from_numpy(wl.page_ids).to(dev)
    s_ids_np, s_offs_np, _ = ops.dest_order(wl.page_ids, wl.slot_offsets)
    s_ids = torch.from_numpy(s_ids_np.astype(np.int32)).to(dev)
    s_offs = torch.from_numpy(s_offs_np).to(dev)
    scale = n_id / wl.n_pages
    out["gather_identity_GBps"] = round(
        scale * timed(lambda: ops.gather(table, ident, offs[:n_id], st)), 1)
    out["scatter_identity_GBps"] = round(
        scale * timed(lambda: ops.scatter(table, ident, offs[:n_id], st)), 1)
    out["gather_cfg2_GBps"] = timed(lambda: ops.gather(table, ids, offs, st))
    out["scatter_cfg2_GBps"] = timed(lambda: ops.scatter(table, s_ids, s_offs, st))
    del full, caches, table, st
    torch.cuda.empty_cache()
    return out


def bench_ceilings(torch, dev, nbytes: int = 16 << 30, reps: int = 5) -> dict:
    """Plain streams over `nbytes` buffers (daser_amd/csrc/bw_probe.hip):
    read-only, write-only and copy, one workgroup per unit of 4 to 64 KiB
    at 1 to 16 workgroups per CU; best HIP-event time of `reps`
    launches each. write_random writes the same units at randomly permuted
    places (the placement of a load's destination pages). Bytes counted: read or written once (copy: both). The
    harmonic mean of the best read and write rates is what a copy that
    alternates the two directions at those rates would sustain."""
    import ctypes

    lib = ctypes.CDLL(os.path.join(ROOT, "daser_amd", "libdaser_bwprobe.so"))
    fn = lib.dsr_bw_probe
    fn.argtypes = [ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64,
                   ctypes.c_int64, ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p]
    fn.restype = ctypes.c_int
    a = torch.empty(nbytes, dtype=torch.uint8, device=dev).fill_(1)
    b = torch.empty(nbytes, dtype=torch.uint8, device=dev).fill_(2)
    sink = torch.zeros(256, dtype=torch.int32, device=dev)
    stream = torch.cuda.current_stream(dev).cuda_stream
    out = {}
    perms = {}
    for op, name in ((0, "read"), (1, "write"), (2, "copy"), (3, "write_random"),
                     (4, "write_random_16_per_wg")):
        moved = nbytes * (2 if op == 2 else 1)
        sweep = []
        for unit in (4 << 10, 8 << 10, 16 << 10, 32 << 10, 64 << 10):
            if op == 3:  # the same units written at randomly permuted places
                g = torch.Generator().manual_seed(unit)
                perms[unit] = torch.randperm(nbytes // unit, generator=g,
                                             dtype=torch.int32).to(dev)
            for wpc in (1, 2, 4, 8, 16):
                def launch():
                    s_ptr = perms[unit].data_ptr() if op >= 3 else a.data_ptr()
                    rc = fn(op, s_ptr, b.data_ptr(), nbytes, unit, wpc, sink.data_ptr(),
                            stream)
                    if rc:
                        raise RuntimeError(f"dsr_bw_probe failed with {rc}")
                launch()
                t = Timer(torch)
                for _ in range(reps):
                    with t:
                        launch()
                torch.cuda.synchronize()
                ms = min(s_.elapsed_time(e_) for s_, e_ in t.pairs)
                sweep.append({"unit_kib": unit >> 10, "wg_per_cu": wpc, "ms": round(ms, 4),
                              "GBps": round(moved / (ms * 1e-3) / 1e9, 1)})
        best = max(sweep, key=lambda r: r["GBps"])
        out[name] = {"best_GBps": best["GBps"], "frac": round(best["GBps"] / HBM_PEAK_GBS, 4),
                     "unit_kib": best["unit_kib"], "wg_per_cu": best["wg_per_cu"],
                     "sweep": sweep}
    del perms
    r, w = out["read"]["best_GBps"], out["write"]["best_GBps"]
    out["read_write_harmonic_GBps"] = round(2 / (1 / r + 1 / w), 1)
    del a, b
    torch.cuda.empty_cache()
    return out


def bench_reuse(torch, ops, position, dev, steps: int = 6) -> list:
    """RAG loads at the Llama-3-8B shape with more or fewer requests sharing
    the cached chunks (10 chunks of 512 tokens per request, n_src distinct
    ones): the fan-out load (ops' path for host tables with shared records)
    against the per-page re-rotation of the same pages, medians of HIP-event
    times."""
    from daser_amd import workloads

    shape = workloads.LLAMA3_8B

    def timed(fn):
        fn()
        t = Timer(torch)
        for _ in range(steps):
            with t:
                fn()
        torch.cuda.synchronize()
        return float(np.median([s_.elapsed_time(e_) for s_, e_ in t.pairs]))

    out = []
    for n_req, n_src in ((2, 16), (3, 16), (4, 20), (8, 16), (16, 16), (32, 160), (32, 64),
                         (32, 40), (32, 20)):
        wl = workloads.rag_reuse(shape, n_req, 10, 512, n_src, 32768, seed=1, pool_slack=1.05)
        full, caches, _ = fill_caches(torch, shape, wl.num_blocks, "bf16", dev, seed=2)
        table = ops.LayerTable(caches)
        src = torch.empty(wl.meta["src_staging_bytes"], dtype=torch.uint8, device=dev)
        src.view(torch.bfloat16).normal_()
        ridx, uniq = position.page_rope_index(wl.chunk_pages, wl.chunk_delta)
        tabs = position.delta_tables(uniq, shape.head_dim, THETA, device=dev)
        ids, offs, rd = ops.dest_order(wl.page_ids, wl.src_offsets, ridx)
        prep = ops.PreparedFanout(table, ids, offs, src, rope=(rd, tabs, None, "neox", None, None))
        ids_d = torch.from_numpy(ids.astype(np.int32)).to(dev)
        offs_d = torch.from_numpy(offs).to(dev)
        rd_d = torch.from_numpy(rd.astype(np.int32)).to(dev)
        per_page = timed(lambda: ops.scatter_rerotate(table, ids_d, offs_d, src, tabs, rd_d,
                                                      shared_records=False))
        fan = timed(prep)
        out.append({"requests": n_req, "cached_chunks": n_src, "pages": wl.n_pages,
                    "placements_per_record": round(wl.n_pages / prep.n_src, 2),
                    "fanout_ms": round(fan, 4), "per_page_ms": round(per_page, 4),
                    "speedup": round(per_page / fan, 3)})
        del full, caches, table, src, prep
        torch.cuda.empty_cache()
    return out


def cpu_model() -> str:
    """The host CPU as /proc/cpuinfo names it: model name verbatim, with its
    family / model / stepping numbers and the logical CPUs listed there."""
    fields, n = {}, 0
    try:
        for line in open("/proc/cpuinfo"):
            key, _, val = line.partition(":")
            key = key.strip()
            if key == "processor":
                n += 1
            elif key in ("model name", "cpu family", "model", "stepping") and key not in fields:
                fields[key] = val.strip()
    except OSError:
        return "unknown"
    return (f"{fields.get('model name', 'unknown')} (family {fields.get('cpu family', '?')}, "
            f"model {fields.get('model', '?')}, stepping {fields.get('stepping', '?')}; "
            f"{n} logical CPUs in /proc/cpuinfo)")


def reference_loop(torch, dev, budget_s: float = 6.0) -> dict:
    """The reference's own copy path, timed on `dev` (the GPU, or "cpu"):
    save = for each page, for each layer,
        staging[off:off+n].copy_(kv[:, b].reshape(-1).view(uint8))
    (daser/connector/daser_connector.py:625-632), load = for each page and
    layer kv[:, b].copy_(staging[off:off+n].view(dtype).view(shape)) (:536-551),
    over 256 Llama-3-8B pages of a 1024-block pool, repeated to ~budget_s."""
    from daser_amd import workloads

    shape = workloads.LLAMA3_8B
    wl = workloads.ragged(shape, 4, 1024, 1024, seed=0, num_blocks=1024)
    kv = [torch.zeros((2, 1024, 16, 8, 128), dtype=torch.bfloat16, device=dev)
          for _ in range(shape.num_layers)]
    staging = torch.empty(wl.staging_bytes, dtype=torch.uint8, device=dev)
    layer = shape.layer_bytes
    blocks = wl.page_ids.tolist()
    offs = wl.slot_offsets.tolist()

    def save():
        for b, o in zip(blocks, offs):
            for l, t in enumerate(kv):
                src = t[:, b]
                staging[o + l * layer:o + l * layer + src.nbytes].copy_(
                    src.reshape(-1).view(torch.uint8))

    def load():
        for b, o in zip(blocks, offs):
            for l, t in enumerate(kv):
                dst = t[:, b]
                dst.copy_(staging[o + l * layer:o + l * layer + dst.nbytes]
                          .view(t.dtype).view(dst.shape))

    sync = torch.cuda.synchronize if dev.type == "cuda" else (lambda: None)
    save()
    load()
    sync()
    n, t0 = 0, time.perf_counter()
    while True:
        save()
        load()
        sync()
        n += 1
        el = time.perf_counter() - t0
        if el >= budget_s:
            break
    P = wl.payload_bytes
    return {"GBps": round(4 * P * n / el / 1e9, 2), "step_ms": round(el / n * 1e3, 2),
            "sample": f"{wl.n_pages} pages x 32 layers, {n} save+load rounds in {el:.1f} s"}


# the re-rotation kernel each configuration's launch selects (by page size)
ROT_KERNEL = {3: "kv_scatter_rerotate_grouped_kernel", 5: "kv_scatter_rerotate_grouped_kernel",
              6: "kv_scatter_rerotate_grouped_kernel"}


def frac_hbm(traffic, ms):
    """HBM fraction on counter bytes: recorded traffic per launch (FETCH_SIZE
    + WRITE_SIZE, scaled) / this run's kernel time / 8 TB/s. Below the
    algorithmic fraction where caches (the memory-side cache) serve part of
    the reads. None if the traffic is not recorded."""
    if traffic is None or not ms:
        return None
    return round(traffic / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)


def pmc_traffic(kernel: str, config: int, pages: int):
    """HBM bytes per launch recorded from rocprofv3 PMC runs of this same
    workload (profiles/pmc_traffic.txt), or None if not recorded."""
    path = os.path.join(ROOT, "profiles", "pmc_traffic.txt")
    if not os.path.exists(path):
        return None
    for line in open(path):
        f = line.split()
        if len(f) == 8 and not line.startswith("#") and f[0] == kernel \
                and int(f[1]) == config and int(f[2]) == pages:
            return int(f[7])
    return None


def cpu_port(budget_s: float = 8.0) -> dict:
    """C oracle (single thread) gather+scatter on a sample of config 2's
    shape: 256 pages of a 1024-block host pool, repeated to ~budget_s."""
    from daser_amd import workloads
    from oracle import oracle

    shape = workloads.LLAMA3_8B
    wl = workloads.ragged(shape, 4, 1024, 1024, seed=0, num_blocks=1024)
    layers = [np.full((2, 1024, 16, 8, 128), 0x3F80 + l, dtype=np.uint16)
              for l in range(shape.num_layers)]
    staging = np.zeros(wl.staging_bytes, dtype=np.uint8)
    P = wl.payload_bytes
    n = 0
    t0 = time.perf_counter()
    while True:
        oracle.gather(layers, wl.page_ids, wl.slot_offsets, staging, shape.layer_bytes)
        oracle.scatter(layers, wl.page_ids, wl.slot_offsets, staging, shape.layer_bytes)
        n += 1
        el = time.perf_counter() - t0
        if el >= budget_s:
            break
    return {
        "value": 4 * P * n / el / 1e9,
        "unit": "GB/s",
        "cores": 1,
        "kind": "port",
        "sample": f"C oracle gather+scatter, {wl.n_pages} pages (256 x 2 MiB records, "
                  f"Llama-3-8B shape) x {n} repetitions in {el:.1f} s, one thread",
    }


def cpu_rerotate(torch, budget_s: float = 8.0) -> dict:
    """fp32 torch rotate-half re-rotation on the host, vectorised: one reused
    512-token chunk of config 3's shape (32 pages x 32 layers) loaded from
    its records into a host cache, V copied and K rotated by one delta
    (neox, theta 5e5), on all host threads; repeated to ~budget_s."""
    from daser_amd import position, workloads

    shape = workloads.LLAMA3_8B
    L, bs, H, D = shape.num_layers, shape.block_size, shape.num_heads, shape.head_dim
    n_pages, nb = 32, 256
    g = torch.Generator().manual_seed(5)
    recs = torch.randn(n_pages, L, 2, bs, H, D, generator=g).to(torch.bfloat16)
    caches = [torch.zeros(2, nb, bs, H, D, dtype=torch.bfloat16) for _ in range(L)]
    dst = torch.randperm(nb, generator=g)[:n_pages]
    cs = position.delta_tables([12345], D, THETA)[0]  # [D/2, 2] float32
    cos = torch.cat([cs[:, 0], cs[:, 0]])
    sin = torch.cat([cs[:, 1], cs[:, 1]])

    def once():
        for l in range(L):
            k = recs[:, l, 0].float()
            rot = torch.cat([-k[..., D // 2:], k[..., :D // 2]], dim=-1)
            caches[l][0, dst] = (k * cos + rot * sin).to(torch.bfloat16)
            caches[l][1, dst] = recs[:, l, 1]

    once()
    n = 0
    t0 = time.perf_counter()
    while True:
        once()
        n += 1
        el = time.perf_counter() - t0
        if el >= budget_s:
            break
    return {"value": n_pages * bs * n / el, "unit": "tokens/s",
            "cores": torch.get_num_threads(), "kind": "torch fp32 rotate-half",
            "sample": f"one 512-token chunk (32 pages x 32 layers, Llama-3-8B shape) x {n} "
                      f"in {el:.1f} s"}


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--configs", default="2,3,4,5,6")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-ref-loop", action="store_true",
                    help="skip timing the reference's per-page torch copy loop on the GPU")
    ap.add_argument("--io", action="store_true",
                    help="also time the PCIe/file-inclusive save and load of the "
                         "connector's data plane on a 2 GiB sample")
    ap.add_argument("--serving", action="store_true",
                    help="also time the connector's worker hooks on serving-shaped "
                         "steps (host cost per hook, save and load latency)")
    ap.add_argument("--patterns", action="store_true",
                    help="also time config 2's bytes in other patterns: torch's copy_, "
                         "index_copy_ and index_select, and this library's kernels over "
                         "the identity page list")
    ap.add_argument("--shapes", action="store_true",
                    help="also time gather, scatter and re-rotation at the cache shapes "
                         "of other model families (MODEL_SHAPES)")
    ap.add_argument("--calibrate", action="store_true",
                    help="also run a plain 4 GiB device copy (the reference kernel "
                         "for scaling rocprofv3 FETCH_SIZE / WRITE_SIZE counters)")
    ap.add_argument("--ceilings", action="store_true",
                    help="also time plain read-only, write-only and copy streams of 16 GiB "
                         "(libdaser_bwprobe.so) over unit sizes and workgroups per CU: what "
                         "the memory system sustains per direction of traffic")
    ap.add_argument("--reuse", action="store_true",
                    help="also time RAG loads with more or fewer requests sharing the cached "
                         "chunks: the fan-out load against the per-page re-rotation")
    ap.add_argument("--no-ceilings", action="store_true",
                    help="skip the short read/write/copy stream measurement that the default "
                         "run adds beside the roofline (hbm_ceilings)")
    ap.add_argument("--tune", default="",
                    help="launch-shape overrides for a measurement, as knob=value pairs "
                         "separated by commas (daser_amd._lib.TUNE names); the bytes moved "
                         "are the same")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: the KV path shards per rank with no "
              "exchange, so --gpus must be 1", file=sys.stderr)
        return 2

    import torch

    from daser_amd import ops, position, workloads

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    if args.tune:
        from daser_amd import _lib

        for kv in args.tune.split(","):
            k, v = kv.split("=")
            _lib.set_tuning(k.strip(), v.strip() if k.strip() == "rot_kernel" else int(v))
        log(f"[bench] tuning overrides: {args.tune}")
    configs = [int(c) for c in args.configs.split(",") if c]
    res = {}
    if args.calibrate:
        n = 4 << 30
        a = torch.empty(n, dtype=torch.uint8, device=dev).fill_(1)
        b = torch.empty_like(a)
        for _ in range(2):
            b.copy_(a)
        torch.cuda.synchronize()
        del a, b
        torch.cuda.empty_cache()
        log(f"[bench] calibration: 2 plain copies of {n} bytes")
    for c in configs:
        log(f"[bench] config {c}: {workloads.CONFIG_NAMES[c]}")
        wl = workloads.config(c)
        if c in (2, 4):
            res[c] = bench_copy(torch, ops, wl, "bf16" if c == 2 else "fp8", dev,
                                args.steps, args.warmup, position)
        else:
            res[c] = bench_rerotate(torch, ops, position, wl, "bf16", dev,
                                    args.steps, args.warmup)
        log(f"[bench] config {c}: {json.dumps(res[c])}")

    out = {"metric": METRIC, "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
           "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
           "data": "synthetic (seeded N(0,1) bf16 KV, seeded random block permutation)"}
    if 2 in res:
        r = res[2]
        out.update({
            "value": round(r["step_GBps"], 1),
            "unit": "GB/s",
            "ms_per_step": round(r["step_ms"], 3),
            "dtype": "u8",
            "config": {"workload": workloads.CONFIG_NAMES[2], "kv_dtype": "bf16",
                       "pages": r["pages"], "tokens": r["tokens"],
                       "payload_bytes_per_pass": r["payload_bytes"]},
        })
        dom = "gather" if r["gather_ms"] >= r["scatter_ms"] else "scatter"
        achieved = r[f"{dom}_GBps"]
        # the one-unit kernels the launch policy picks for 32 KiB pages
        kname = "kv_gather_kernel" if dom == "gather" else "kv_scatter_stream_kernel"
        out["roofline"] = {
            "kernel": kname,
            "bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
            "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": pmc_traffic(kname, 2, r["pages"]),
            "algorithmic_bytes": 2 * r["payload_bytes"],
        }
        out["kernels"] = {
            "gather": {"ms": round(r["gather_ms"], 4), "GBps": round(r["gather_GBps"], 1),
                       "frac": round(r["gather_GBps"] / HBM_PEAK_GBS, 4)},
            "scatter": {"ms": round(r["scatter_ms"], 4), "GBps": round(r["scatter_GBps"], 1),
                        "frac": round(r["scatter_GBps"] / HBM_PEAK_GBS, 4)},
        }
        out["kernels"]["gather_slots"] = {
            "ms": round(r["slots_gather_ms"], 4), "GBps": round(r["slots_gather_GBps"], 1),
            "frac": round(r["slots_gather_GBps"] / HBM_PEAK_GBS, 4)}
        split = (f"{r['slots_whole_pages']} whole pages through the page kernel, "
                 f"{r['slots_ragged_tokens']} ragged-edge tokens through the token kernel")
        out["kernels"]["scatter_slots"] = {
            "ms": round(r["slots_scatter_ms"], 4), "GBps": round(r["slots_scatter_GBps"], 1),
            "frac": round(r["slots_scatter_GBps"] / HBM_PEAK_GBS, 4),
            "path": "kv_scatter_stream_kernel + kv_slots_kernel: " + split}
        out["kernels"]["scatter_slots_rerotate"] = {
            "ms": round(r["slots_rerotate_ms"], 4), "GBps": round(r["slots_rerotate_GBps"], 1),
            "frac": round(r["slots_rerotate_GBps"] / HBM_PEAK_GBS, 4),
            "path": "kv_scatter_rerotate_grouped_kernel + kv_slots_rerotate_kernel: " + split}
        out["check"] = {"round_trip_probe": r["probe_ok"]}
    for c in (3, 5, 6):
        if c in res:
            r = res[c]
            out[f"rerotate_cfg{c}"] = {
                "workload": workloads.CONFIG_NAMES[c],
                "tokens_per_s": round(r["tokens_per_s"]),
                "GBps": round(r["GBps"], 1), "frac": round(r["frac_hbm_peak"], 4),
                "kernel_ms": round(r["kernel_ms"], 4), "tokens": r["tokens"],
                "same_pages_plain_scatter_GBps": round(r["plain_scatter_GBps"], 1),
                "split_x_k_layout_GBps": round(r["kx_GBps"], 1),
                **({"same_pages_gather_GBps": round(r["gather_GBps"], 1)}
                   if "gather_GBps" in r else {}),
                **({"same_pages_slots_gather_GBps": round(r["slots_gather_GBps"], 1),
                    "same_pages_slots_scatter_GBps": round(r["slots_scatter_GBps"], 1)}
                   if "slots_gather_GBps" in r else {}),
                "kernel": ROT_KERNEL[c],
                "traffic": pmc_traffic(ROT_KERNEL[c], c, r["pages"]),
                "algorithmic_bytes": 2 * r["payload_bytes"]}
            out[f"rerotate_cfg{c}"]["frac_hbm"] = frac_hbm(
                out[f"rerotate_cfg{c}"]["traffic"], r["kernel_ms"])
            if "fanout_ms" in r:
                # the load the library runs for these host tables: each shared
                # record read once (reads: the distinct records; writes: P)
                per_page = {k: out[f"rerotate_cfg{c}"].pop(k) for k in
                            ("tokens_per_s", "GBps", "frac", "kernel_ms", "kernel", "traffic",
                             "algorithmic_bytes", "frac_hbm")}
                alg = r["fanout_read_bytes"] + r["payload_bytes"]
                fms = r["fanout_ms"]
                out[f"rerotate_cfg{c}"].update({
                    "tokens_per_s": round(r["tokens"] / (fms * 1e-3)),
                    "GBps": round(alg / (fms * 1e-3) / 1e9, 1),
                    "frac": round(alg / (fms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                    "kernel_ms": round(fms, 4), "kernel": "kv_fanout_kernel",
                    "algorithmic_bytes": alg,
                    "traffic": pmc_traffic("kv_fanout_kernel", c, r["pages"]),
                    "distinct_records": r["fanout_sources"],
                    "same_pages_plain_fanout_GBps": round(
                        alg / (r["fanout_plain_ms"] * 1e-3) / 1e9, 1),
                    "per_page_path": per_page})
                out[f"rerotate_cfg{c}"]["frac_hbm"] = frac_hbm(
                    out[f"rerotate_cfg{c}"]["traffic"], fms)
    if 4 in res:
        r = res[4]
        out["fp8_cfg4"] = {"workload": workloads.CONFIG_NAMES[4],
                           "gather_GBps": round(r["gather_GBps"], 1),
                           "scatter_GBps": round(r["scatter_GBps"], 1),
                           "gather_ms": round(r["gather_ms"], 4),
                           "scatter_ms": round(r["scatter_ms"], 4),
                           "rerotate_GBps": round(r.get("rerotate_GBps", 0.0), 1),
                           "rerotate_tokens_per_s": round(r.get("rerotate_tokens_per_s", 0.0)),
                           "rerotate_ms": round(r.get("rerotate_ms", 0.0), 4),
                           "rerotate_e5m2_GBps": round(r.get("rerotate_e5m2_GBps", 0.0), 1),
                           "tokens": r["tokens"], "payload_bytes": r["payload_bytes"],
                           "traffic_rerotate": pmc_traffic("kv_scatter_rerotate_contig_kernel", 4,
                                                           r["pages"])}
        f8 = out["fp8_cfg4"]
        f8["frac"] = {k: round(r[f"{k}_GBps"] / HBM_PEAK_GBS, 4)
                      for k in ("gather", "scatter", "rerotate") if r.get(f"{k}_GBps")}
        f8["frac_hbm"] = {
            "gather": frac_hbm(pmc_traffic("kv_gather_kernel", 4, r["pages"]), r["gather_ms"]),
            "scatter": frac_hbm(pmc_traffic("kv_scatter_kernel", 4, r["pages"]), r["scatter_ms"]),
            "rerotate": frac_hbm(f8["traffic_rerotate"], r.get("rerotate_ms"))}
    if "value" not in out and configs:
        r = res[configs[0]]
        out.update({"value": round(r.get("tokens_per_s", 0.0)), "unit": "tokens/s",
                    "ms_per_step": round(r.get("kernel_ms", 0.0), 3), "dtype": "bf16",
                    "config": {"workload": workloads.CONFIG_NAMES[configs[0]]}})
    if args.ceilings or (2 in res and not args.no_ceilings):
        log("[bench] ceilings: plain read, write and copy streams")
        ceil = bench_ceilings(torch, dev)
        if args.ceilings:
            out["ceilings"] = ceil
            log(f"[bench] ceilings: {json.dumps(ceil)}")
        bound = ceil["read_write_harmonic_GBps"]
        out["hbm_ceilings"] = {
            "read_GBps": ceil["read"]["best_GBps"], "write_GBps": ceil["write"]["best_GBps"],
            "copy_bound_GBps": bound, "plain_copy_GBps": ceil["copy"]["best_GBps"],
            "write_random_GBps": ceil["write_random"]["best_GBps"],
            "write_random_16_per_wg_GBps": ceil["write_random_16_per_wg"]["best_GBps"],
            "note": "measured on this GPU in this run (libdaser_bwprobe.so streams); a copy "
                    "moves as many bytes each way, so it is bounded near the harmonic mean "
                    "of the read and write rates"}
        if "roofline" in out:
            out["roofline"]["frac_of_copy_bound"] = round(out["roofline"]["achieved"] / bound, 4)
    if args.reuse:
        log("[bench] reuse: fan-out against per-page loads by chunk sharing")
        out["reuse"] = bench_reuse(torch, ops, position, dev)
        log(f"[bench] reuse: {json.dumps(out['reuse'])}")
    if args.patterns:
        log("[bench] patterns: config 2's bytes in other access patterns")
        out["patterns"] = bench_patterns(torch, ops, dev)
        log(f"[bench] patterns: {json.dumps(out['patterns'])}")
    if args.shapes:
        log("[bench] shapes: other model families' caches")
        out["shapes"] = bench_shapes(torch, ops, position, dev)
    if args.io:
        log("[bench] io: PCIe/file-inclusive save and load")
        out["pcie_inclusive"] = bench_io(torch, dev)
        log(f"[bench] io: {json.dumps(out['pcie_inclusive'])}")
    if args.serving:
        log("[bench] serving: connector worker hooks per step")
        out["serving"] = bench_serving(torch, dev)
        log(f"[bench] serving: {json.dumps(out['serving'])}")
    if not args.no_ref_loop:
        log("[bench] reference copy loop on the GPU")
        out["reference_loop_gpu"] = reference_loop(torch, dev)
    if not args.no_cpu:
        ncpu = len(os.sched_getaffinity(0))
        torch.set_num_threads(ncpu)
        log(f"[bench] cpu baseline: the reference's copy loops in torch on the CPU "
            f"({ncpu} threads)")
        r = reference_loop(torch, torch.device("cpu"), budget_s=12.0)
        out["cpu_baseline"] = {
            "value": r["GBps"], "unit": "GB/s", "cores": ncpu, "kind": "reference torch loop",
            "cpu_model": cpu_model(),
            "sample": "torch restatement of daser_connector.py:625-632 (save: reshape + copy_ "
                      "per page and layer) and :536-551 (load: copy_ per page and layer) on "
                      f"host tensors, {torch.get_num_threads()} torch threads; {r['sample']}"}
        log("[bench] C oracle gather+scatter on the CPU (one thread)")
        out["cpu_port"] = cpu_port()
        log(f"[bench] fp32 torch re-rotation on the CPU ({ncpu} threads)")
        out["cpu_rerotate"] = cpu_rerotate(torch)
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
