"""Host logic of the connector (no GPU): page planning, the scheduler role
against a fake IPC client, and the pinned-ring store I/O run on CPU tensors
(ordering, slow and failing I/O, short reads)."""

from __future__ import annotations

import asyncio
import os
import threading
import time
from types import SimpleNamespace

import numpy as np
import pytest
import torch

from daser_amd import connector as C
from daser_amd.store_io import PinnedRingIO, StoreIOError, preallocate_store

SLOT = 4096


def test_plan_store_layout_matches_reference_offsets():
    reqs = {
        "a": C.ReqStoreSpec("ka", start_slot=10, num_slots=3, block_ids=[7, 2, 5],
                            file_offset=10 * SLOT, token_count=48),
        "empty": C.ReqStoreSpec("ke", 0, 0, [], 0, 0),
        "b": C.ReqStoreSpec("kb", start_slot=3, num_slots=1, block_ids=[9],
                            file_offset=3 * SLOT, token_count=16),
    }
    p = C.plan_store(reqs, SLOT)
    assert p.page_ids.tolist() == [7, 2, 5, 9]
    assert p.slot_offsets.tolist() == [0, SLOT, 2 * SLOT, 3 * SLOT]
    # one transfer per request at start_slot * SLOT (reference :652)
    assert p.transfers == [("ka", 0, 3 * SLOT, 10 * SLOT), ("kb", 3 * SLOT, SLOT, 3 * SLOT)]
    assert p.arena_bytes == 4 * SLOT


def test_coalesce_transfers_merges_file_neighbours():
    from daser_amd.data_plane import coalesce_transfers

    t = [("a", 0, 3 * SLOT, 10 * SLOT), ("b", 3 * SLOT, SLOT, 13 * SLOT),
         ("c", 4 * SLOT, 2 * SLOT, 2 * SLOT), ("d", 6 * SLOT, SLOT, 4 * SLOT),
         ("e", 7 * SLOT, SLOT, 20 * SLOT)]
    assert coalesce_transfers(t) == [(["a", "b"], 0, 4 * SLOT, 10 * SLOT),
                                     (["c", "d"], 4 * SLOT, 3 * SLOT, 2 * SLOT),
                                     (["e"], 7 * SLOT, SLOT, 20 * SLOT)]
    assert coalesce_transfers([]) == []


def test_plan_load_without_positions_is_plain_scatter():
    reqs = {"r": C.ReqLoadSpec("k", start_slot=4, num_slots=2, block_ids=[11, 3],
                               file_offset=4 * SLOT, token_count=20)}
    p = C.plan_load(reqs, SLOT)
    assert p.page_ids.tolist() == [11, 3]
    assert p.src_offsets.tolist() == [0, SLOT]
    assert p.rope_idx.tolist() == [-1, -1] and p.deltas == []
    assert p.reads == [(0, 2 * SLOT, 4 * SLOT)]


def test_plan_load_positions_and_segments():
    reqs = {
        "r1": C.ReqLoadSpec("k1", 0, 2, [1, 2], 0, 32, pos_offset=100, new_pos=612),
        "r2": C.ReqLoadSpec("k2", 0, 0, [5, 6, 7], 0, 48, segments=[
            C.LoadSegment(start_slot=20, num_slots=2, block_offset=0, pos_offset=0, new_pos=512),
            C.LoadSegment(start_slot=8, num_slots=1, block_offset=2, pos_offset=0, new_pos=0),
        ]),
        "r3": C.ReqLoadSpec("k3", 0, 1, [9], 0, 16, pos_offset=7, new_pos=7),
    }
    p = C.plan_load(reqs, SLOT)
    assert p.page_ids.tolist() == [1, 2, 5, 6, 7, 9]
    assert p.deltas == [512]  # 612 - 100 and 512 - 0 share one table
    assert p.rope_idx.tolist() == [0, 0, 0, 0, -1, -1]
    # r3's slot 0 lies inside r1's read of slots 0-1: no read of its own
    assert p.reads == [(0, 2 * SLOT, 0), (2 * SLOT, 2 * SLOT, 20 * SLOT),
                       (4 * SLOT, SLOT, 8 * SLOT)]
    assert p.src_offsets.tolist() == [0, SLOT, 2 * SLOT, 3 * SLOT, 4 * SLOT, 0]
    assert p.page_read.tolist() == [0, 0, 1, 1, 2, 0] and p.shared_records
    with pytest.raises(ValueError):
        C.plan_load({"x": C.ReqLoadSpec("k", 0, 0, [1], 0, 16, segments=[
            C.LoadSegment(0, 2, 0)])}, SLOT)


def test_plan_load_reads_a_shared_chunk_once():
    """Requests hitting the same cached chunk (or a part of one already read)
    read it once; each scatters from that read into its own blocks, at its
    own position."""
    reqs = {
        "a": C.ReqLoadSpec("k", 6, 4, [10, 11, 12, 13], 6 * SLOT, 64, pos_offset=0,
                           new_pos=100),
        "b": C.ReqLoadSpec("k", 6, 4, [20, 21, 22, 23], 6 * SLOT, 64, pos_offset=0,
                           new_pos=900),
        "c": C.ReqLoadSpec("k2", 0, 0, [30, 31], 0, 32, segments=[
            C.LoadSegment(start_slot=8, num_slots=2, block_offset=0)]),  # inside a's read
        "d": C.ReqLoadSpec("k3", 9, 2, [40, 41], 9 * SLOT, 32),  # overlaps, not inside
    }
    p = C.plan_load(reqs, SLOT)
    assert p.reads == [(0, 4 * SLOT, 6 * SLOT), (4 * SLOT, 2 * SLOT, 9 * SLOT)]
    assert p.arena_bytes == 6 * SLOT
    assert p.page_ids.tolist() == [10, 11, 12, 13, 20, 21, 22, 23, 30, 31, 40, 41]
    assert p.src_offsets.tolist() == [0, SLOT, 2 * SLOT, 3 * SLOT] * 2 + \
        [2 * SLOT, 3 * SLOT, 4 * SLOT, 5 * SLOT]
    assert p.rope_idx.tolist() == [0] * 4 + [1] * 4 + [-1] * 4 and p.deltas == [100, 900]
    assert p.page_read.tolist() == [0] * 10 + [1, 1] and p.shared_records
    alone = C.plan_load({"a": reqs["a"], "d": reqs["d"]}, SLOT)
    assert not alone.shared_records and len(alone.reads) == 2


def test_plan_load_block_targeted_twice_keeps_the_last_load():
    """The reference's sequential copies leave the last load's bytes in a
    block that two loads of a step target; the plan keeps that load only,
    whatever order its read batches scatter in."""
    reqs = {
        "x": C.ReqLoadSpec("ka", 5, 2, [3, 9], 5 * SLOT, 32),
        "y": C.ReqLoadSpec("kb", 20, 2, [9, 4], 20 * SLOT, 32, pos_offset=0, new_pos=64),
        "z": C.ReqLoadSpec("ka", 5, 2, [4, 11], 5 * SLOT, 32),  # reuses x's read
    }
    p = C.plan_load(reqs, SLOT)
    assert p.page_ids.tolist() == [3, 9, 4, 11]
    assert p.src_offsets.tolist() == [0, 2 * SLOT, 0, SLOT]
    assert p.rope_idx.tolist() == [-1, 0, -1, -1]
    assert p.page_read.tolist() == [0, 1, 0, 0]


def test_dest_order_keeps_the_last_entry_of_a_block():
    from daser_amd import ops

    ids, offs, extra = ops.dest_order([7, 2, 7, 5, 2, 7], [0, 16, 32, 48, 64, 80],
                                      [1, 2, 3, 4, 5, 6])
    assert ids.tolist() == [2, 5, 7]
    assert offs.tolist() == [64, 48, 80]
    assert extra.tolist() == [5, 4, 6]


# ---------------------------------------------------------------- scheduler


class FakeIPC:
    def __init__(self, chunks=None, alloc=None, fail=False):
        self.chunks, self.alloc, self.fail, self.calls = chunks or [], alloc, fail, []

    def match_and_alloc(self, prefix, store_key, model_id):
        self.calls.append((list(prefix), store_key, model_id))
        if self.fail:
            raise ConnectionError("server down")
        return {"chunks": self.chunks, "alloc": self.alloc}


def _cfg(**extra):
    return SimpleNamespace(kv_transfer_config=SimpleNamespace(kv_connector_extra_config=extra))


def _req(rid, n):
    return SimpleNamespace(request_id=rid, prompt_token_ids=list(range(n)))


def _blocks(ids):
    return SimpleNamespace(blocks=[[SimpleNamespace(block_id=i) for i in ids]])


def test_scheduler_hit_carries_positions():
    """The reference's prefix hit (one chunk, matching the prompt from token
    0) is placed at position 0, so a chunk stored at another position
    (pos_offset 3000) is re-rotated back to 0 on load."""
    chunk = {"chunk_key": "ck", "start_slot": 5, "num_slots": 3, "file_offset": 5 * SLOT,
             "token_count": 40, "pos_offset": 3000}
    ipc = FakeIPC(chunks=[chunk])
    conn = C.DaserConnector(_cfg(block_tokens=16), C.KVConnectorRole.SCHEDULER, ipc_client=ipc)
    n, is_async = conn.get_num_new_matched_tokens(_req("r", 50), 0)
    assert (n, is_async) == (40, False)
    assert len(ipc.calls[0][0]) == 48  # block-aligned prefix
    conn.update_state_after_alloc(_req("r", 50), _blocks([8, 1, 4, 6]), 40)
    meta = conn.build_connector_meta(SimpleNamespace(num_scheduled_tokens={"r": 50}))
    spec = meta.reqs_to_load["r"]
    assert spec.block_ids == [8, 1, 4]  # ceil(40 / 16)
    assert (spec.pos_offset, spec.new_pos) == (3000, 0)
    assert spec.segments == [] and spec.num_slots == 3 and spec.start_slot == 5
    assert meta.reqs_to_store == {}
    plan = C.plan_load(meta.reqs_to_load, SLOT)
    assert plan.deltas == [-3000] and plan.rope_idx.tolist() == [0, 0, 0]


def test_scheduler_miss_allocates_store():
    alloc = {"chunk_key": "new", "start_slot": 2, "num_slots": 2, "file_offset": 2 * SLOT,
             "token_count": 32}
    conn = C.DaserConnector(_cfg(), C.KVConnectorRole.SCHEDULER, ipc_client=FakeIPC(alloc=alloc))
    assert conn.get_num_new_matched_tokens(_req("r", 40), 0) == (0, False)
    conn.update_state_after_alloc(_req("r", 40), _blocks([3, 9, 4]), 0)
    meta = conn.build_connector_meta(SimpleNamespace(num_scheduled_tokens={"r": 40}))
    assert meta.reqs_to_store["r"].block_ids == [3, 9]
    assert conn.request_finished(_req("r", 40), []) == (False, None)


def test_scheduler_ipc_failure_is_a_miss():
    conn = C.DaserConnector(_cfg(), C.KVConnectorRole.SCHEDULER, ipc_client=FakeIPC(fail=True))
    assert conn.get_num_new_matched_tokens(_req("r", 64), 0) == (0, False)
    assert conn.get_num_new_matched_tokens(_req("s", 8), 0) == (0, False)  # < one block


def test_hash_tokens_deterministic():
    assert C.hash_tokens([1, 2, 3]) == C.hash_tokens([1, 2, 3])
    assert C.hash_tokens([1, 2, 3]) != C.hash_tokens([1, 2, 4])
    assert len(C.hash_tokens([5])) == 32


# ---------------------------------------------------------------- store I/O


@pytest.fixture()
def store(tmp_path):
    path = str(tmp_path / "daser.store")
    preallocate_store(path, 1 << 20)
    return path


def test_preallocate_and_missing_file(tmp_path, store):
    assert os.path.getsize(store) == 1 << 20
    preallocate_store(store, 5)  # existing file untouched
    assert os.path.getsize(store) == 1 << 20
    with pytest.raises(FileNotFoundError):
        PinnedRingIO(str(tmp_path / "nope"), "cpu")


def test_ring_round_trip_more_pieces_than_slots(store):
    rng = np.random.default_rng(0)
    src = torch.from_numpy(rng.integers(0, 256, 100_000, dtype=np.uint8))
    with PinnedRingIO(store, "cpu", slot_bytes=4096, n_slots=3) as io:
        assert io.write_from_device(src, 12_288) == src.numel()
        dst = torch.zeros_like(src)
        assert io.read_into_device(dst, 12_288) == src.numel()
    assert torch.equal(src, dst)
    with open(store, "rb") as f:
        f.seek(12_288)
        assert f.read(100_000) == src.numpy().tobytes()


def test_ring_slow_writer_keeps_order(store):
    """A writer that stalls must not let a slot be overwritten early."""
    def hook(kind, off, n):
        if kind == "write":
            time.sleep(0.01)

    a = torch.full((40_000,), 1, dtype=torch.uint8)
    b = torch.full((40_000,), 2, dtype=torch.uint8)
    with PinnedRingIO(store, "cpu", slot_bytes=4096, n_slots=2, io_hook=hook) as io:
        io.write_from_device(a, 0)
        io.write_from_device(b, 40_000)
        out = torch.zeros(80_000, dtype=torch.uint8)
        io.read_into_device(out, 0)
    assert torch.equal(out[:40_000], a) and torch.equal(out[40_000:], b)


def test_ring_failed_write_raises(store):
    def hook(kind, off, n):
        if kind == "write" and off >= 8192:
            raise OSError("disk full")

    with PinnedRingIO(store, "cpu", slot_bytes=4096, n_slots=2, io_hook=hook) as io:
        with pytest.raises(OSError, match="disk full"):
            io.write_from_device(torch.ones(20_000, dtype=torch.uint8), 0)
        # the ring stays usable for later transfers below the failing range
        io._hook = None
        io.write_from_device(torch.ones(10, dtype=torch.uint8), 0)


def test_ring_short_read_raises(store):
    with PinnedRingIO(store, "cpu", slot_bytes=4096, n_slots=2) as io:
        with pytest.raises(StoreIOError, match="short read"):
            io.read_into_device(torch.zeros(8192, dtype=torch.uint8), (1 << 20) - 100)


def test_ring_async_api_and_close(store):
    io = PinnedRingIO(store, "cpu", slot_bytes=1024, n_slots=2)
    src = torch.arange(5000, dtype=torch.int32)

    async def go():
        await io.write_async(src, 4096)
        dst = torch.zeros_like(src)
        await io.read_into_async(dst, 4096)
        return dst

    assert torch.equal(asyncio.run(go()), src)
    io.close()
    io.close()
    with pytest.raises(StoreIOError):
        io.write_from_device(src, 0)


def test_ring_concurrent_callers_serialise(store):
    """Transfers from two threads do not interleave inside the ring."""
    errs = []

    def work(val, off):
        try:
            t = torch.full((30_000,), val, dtype=torch.uint8)
            for _ in range(5):
                io.write_from_device(t, off)
        except Exception as e:  # pragma: no cover
            errs.append(e)

    with PinnedRingIO(store, "cpu", slot_bytes=2048, n_slots=3) as io:
        th = [threading.Thread(target=work, args=(v, v * 40_000)) for v in (1, 2)]
        [t.start() for t in th]
        [t.join() for t in th]
        out = torch.zeros(80_000, dtype=torch.uint8)
        io.read_into_device(out, 40_000)
    assert not errs
    assert (out[:30_000] == 1).all() and (out[40_000:70_000] == 2).all()


def test_worker_hooks_without_metadata_are_noops(tmp_path):
    """Reference behaviour of the worker hooks with no bound metadata or
    with nothing to load or store: return silently, launch nothing
    (daser_connector.py:455-472, 574-580, 634-640)."""
    from types import SimpleNamespace

    import torch

    from daser_amd import connector as C

    class IPC:
        async def commit_chunk(self, key):
            raise AssertionError("nothing may be committed")

    cfg = SimpleNamespace(kv_transfer_config=SimpleNamespace(kv_connector_extra_config=dict(
        store_path=str(tmp_path / "s"), io_slot_mb=0.03125, io_slots=3, io_backend="python")))
    w = C.DaserConnector(cfg, C.KVConnectorRole.WORKER, ipc_async=IPC())
    caches = {f"model.layers.{i}.self_attn.attn": torch.zeros(2, 16, 16, 2, 64, dtype=torch.bfloat16)
              for i in range(3)}
    w.register_kv_caches(caches)
    layer = caches["model.layers.0.self_attn.attn"]
    for meta in (None, C.DaserConnectorMeta()):
        if meta is not None:
            w.bind_connector_metadata(meta)
        w.start_load_kv(None)
        w.wait_for_layer_load("model.layers.0.self_attn.attn")
        w.save_kv_layer("model.layers.0.self_attn.attn", layer, None)
        w.save_kv_layer("not.a.layer", layer, None)
        w.wait_for_save()
        w.clear_connector_metadata()
    assert (tmp_path / "s").stat().st_size > 0  # store pre-allocated at registration
    w.shutdown()


def test_fp8_rotated_load_needs_k_scales(tmp_path):
    """Re-rotating e4m3 codes needs each layer's K scale: taken from the
    attention modules in forward_context.no_compile_layers, or from the
    extra config; with neither the load raises before any I/O."""
    from types import SimpleNamespace

    import torch

    from daser_amd import connector as C

    def worker(**extra):
        cfg = SimpleNamespace(kv_transfer_config=SimpleNamespace(kv_connector_extra_config=dict(
            store_path=str(tmp_path / "s"), io_backend="python", io_slot_mb=0.03125,
            io_slots=2, **extra)))
        w = C.DaserConnector(cfg, C.KVConnectorRole.WORKER, ipc_async=object())
        names = [f"model.layers.{i}.self_attn.attn" for i in range(3)]
        w.register_kv_caches({n: torch.zeros(2, 8, 16, 1, 64, dtype=torch.float8_e4m3fn)
                              for n in names})
        return w, names

    w, names = worker()
    slot = w._slot_size
    w.bind_connector_metadata(C.DaserConnectorMeta(reqs_to_load={
        "r": C.ReqLoadSpec("k", 0, 1, [2], 0, 16, pos_offset=0, new_pos=100)}))
    with pytest.raises(ValueError, match="K scale"):
        w.start_load_kv(SimpleNamespace(no_compile_layers={}))
    fc = SimpleNamespace(no_compile_layers={
        n: SimpleNamespace(_k_scale=torch.tensor([0.5 + i])) for i, n in enumerate(names)})
    assert torch.equal(w._fp8_k_scales(fc), torch.tensor([0.5, 1.5, 2.5]))
    w.shutdown()
    w2, _ = worker(k_scale=0.25)
    assert torch.equal(w2._fp8_k_scales(None), torch.full((3,), 0.25))
    assert slot == 3 * 2 * 16 * 64
    w2.shutdown()


@pytest.mark.parametrize("cache_dtype,expect", [("fp8", "float8_e4m3fn"),
                                                 ("fp8_e4m3", "float8_e4m3fn"),
                                                 ("fp8_e5m2", "float8_e5m2"),
                                                 ("auto", "uint8")])
def test_uint8_fp8_cache_viewed_as_e4m3(tmp_path, cache_dtype, expect):
    """vLLM may allocate an fp8 cache as uint8; with cache_config.cache_dtype
    fp8 the connector registers an e4m3fn view (no copy)."""
    from types import SimpleNamespace

    import torch

    from daser_amd import connector as C

    cfg = SimpleNamespace(
        cache_config=SimpleNamespace(cache_dtype=cache_dtype),
        kv_transfer_config=SimpleNamespace(kv_connector_extra_config=dict(
            store_path=str(tmp_path / "s"), io_backend="python", io_slot_mb=0.03125,
            io_slots=2)))
    w = C.DaserConnector(cfg, C.KVConnectorRole.WORKER, ipc_async=object())
    t = torch.zeros(2, 8, 16, 1, 64, dtype=torch.uint8)
    w.register_kv_caches({"model.layers.0.self_attn.attn": t})
    assert str(w._plane.table.layout.dtype) == f"torch.{expect}"
    w.shutdown()


def test_stalled_store_io_times_out(tmp_path):
    """A store write or read that does not return raises TimeoutError after
    io_timeout (the reference's worker I/O waits 120 s), forced here with a
    ring whose file writes stall."""
    import threading
    import time

    import torch

    from daser_amd import connector as C
    from daser_amd.store_io import PinnedRingIO

    release = threading.Event()

    def stall(kind, n, off):
        release.wait(5.0)

    caches = {f"model.layers.{i}.self_attn.attn": torch.zeros(2, 8, 16, 1, 64,
                                                              dtype=torch.bfloat16)
              for i in range(2)}
    p = C.KVDataPlane(str(tmp_path / "s"), io_backend="python", io_timeout=0.3, io_readers=1)
    slot = p.register(caches)
    p.io.close()
    p.io = PinnedRingIO(p.store_path, "cpu", slot_bytes=4096, n_slots=2, io_hook=stall)
    plan = C.plan_store({"r": C.ReqStoreSpec("k", 0, 2, [1, 3], 0, 32)}, slot)
    arena = p.new_store_arena(plan)
    t0 = time.monotonic()
    with pytest.raises(TimeoutError, match="store write"):
        p.flush(plan, arena)
    assert time.monotonic() - t0 < 3.0
    lp = C.plan_load({"r": C.ReqLoadSpec("k", 0, 2, [1, 3], 0, 32)}, slot)
    with pytest.raises(TimeoutError, match="store read"):
        p.load(lp)
    release.set()
    p.close()


def test_random_load_plans_cover_shared_reads_and_repeated_blocks():
    """The random plans of the GPU test (tests/test_connector_gpu.py) do
    exercise what they are for: over its seeds, segments served by an
    earlier read, blocks loaded twice in a step, moved and kept positions."""
    from tests.test_connector_gpu import SHAPE, random_load_reqs

    shared = repeated = moved = kept = 0
    for seed in range(12):
        reqs = random_load_reqs(np.random.default_rng(100 + seed), SHAPE.slot_bytes, 40, 48)
        p = C.plan_load(reqs, SHAPE.slot_bytes)
        shared += p.shared_records
        ids = [b for s in reqs.values() for b in s.block_ids]
        repeated += len(set(ids)) < len(ids)
        assert np.unique(p.page_ids).size == p.page_ids.size
        moved += int((p.rope_idx >= 0).any())
        kept += int((p.rope_idx < 0).any())
    assert min(shared, repeated, moved, kept) >= 3, (shared, repeated, moved, kept)


def test_rank_store_path(monkeypatch):
    """One store file per tensor-parallel rank when the path asks for it;
    the rank comes from vLLM when it runs the worker, else the environment."""
    assert C.rank_store_path("/s/daser.store") == "/s/daser.store"
    assert C.rank_store_path("/s/daser.{rank}.store", 3) == "/s/daser.3.store"
    monkeypatch.setenv("LOCAL_RANK", "5")
    assert C.rank_store_path("/s/r{rank}/daser.store") == "/s/r5/daser.store"
    monkeypatch.delenv("LOCAL_RANK")
    monkeypatch.setenv("RANK", "2")
    assert C.rank_store_path("/s/{rank}") == "/s/2"
