"""Worker hooks end to end on the GPU: save_kv_layer / wait_for_save write
the reference's record layout to the store file; start_load_kv reads it back
into other blocks, re-rotating K where the chunk's position changed."""

from __future__ import annotations

from types import SimpleNamespace

import numpy as np
import pytest
import torch

from daser_amd import connector as C
from daser_amd.store_io import NativeRingIO, PinnedRingIO, preallocate_store
from daser_amd.workloads import KVShape
from oracle import oracle
from tests.helpers import rand_caches, to_bits_np

pytestmark = pytest.mark.gpu

SHAPE = KVShape(3, 2, 64, 16, 2)  # SLOT = 3 x 8 KiB


class FakeAsyncIPC:
    def __init__(self):
        self.committed = []

    async def commit_chunk(self, key):
        self.committed.append(key)
        return {"ok": True}


def _worker(tmp_path, **extra):
    cfg = SimpleNamespace(kv_transfer_config=SimpleNamespace(kv_connector_extra_config=dict(
        store_path=str(tmp_path / "daser.store"), io_slot_mb=0.03125, io_slots=3, **extra)))
    ipc = FakeAsyncIPC()
    return C.DaserConnector(cfg, C.KVConnectorRole.WORKER, ipc_async=ipc), ipc


def _named(caches):
    return {f"model.layers.{i}.self_attn.attn": c for i, c in enumerate(caches)}


def _save(w, named, reqs):
    w.bind_connector_metadata(C.DaserConnectorMeta(reqs_to_store=reqs))
    for name, t in named.items():
        w.save_kv_layer(name, t, None)
    w.wait_for_save()
    w.clear_connector_metadata()


def _store_reqs():
    slot = SHAPE.slot_bytes
    return {
        "a": C.ReqStoreSpec("ka", 3, 3, [5, 9, 2], 3 * slot, 40),
        "b": C.ReqStoreSpec("kb", 10, 1, [7], 10 * slot, 16),
    }


def _file_records(path, start_slot, n):
    slot = SHAPE.slot_bytes
    with open(path, "rb") as f:
        f.seek(start_slot * slot)
        return np.frombuffer(f.read(n * slot), dtype=np.uint8)


@pytest.mark.parametrize("mode,backend,stream", [
    ("per_layer", "native", "side"), ("deferred", "native", "side"),
    ("per_layer", "python", "side"), ("per_layer", "native", "current"),
    ("deferred", "python", "current"), ("per_layer", "direct", "side"),
    ("per_layer", "native", "auto-side"), ("per_layer", "native", "auto-current"),
    ("per_layer", "mmap", "side"), ("deferred", "mmap", "current")])
def test_save_writes_reference_layout(gpu, tmp_path, monkeypatch, mode, backend, stream):
    print(f"case: connector save {mode} {backend} {stream}", flush=True)
    if stream.startswith("auto"):
        from daser_amd import data_plane

        # a step's per-layer gather here is 4 pages x 8 KiB: the side stream is
        # chosen when the threshold is below that
        monkeypatch.setattr(data_plane, "SIDE_STREAM_MIN_LAYER_BYTES",
                            1 if stream == "auto-side" else 1 << 40)
        seen = []
        orig = data_plane.KVDataPlane._save_stream
        monkeypatch.setattr(data_plane.KVDataPlane, "_save_stream",
                            lambda self, plan: seen.append(plan.on_side) or orig(self, plan))
    w, ipc = _worker(tmp_path, save_mode=mode, io_backend=backend,
                     save_stream=stream.split("-")[0])
    caches = rand_caches(SHAPE, 16, "bf16", gpu, seed=31)
    named = _named(caches)
    w.register_kv_caches(named)
    assert w._slot_size == SHAPE.slot_bytes
    _save(w, named, _store_reqs())
    host = [to_bits_np(c, "bf16") for c in caches]
    for start, blocks in ((3, [5, 9, 2]), (10, [7])):
        ref = np.zeros(len(blocks) * SHAPE.slot_bytes, dtype=np.uint8)
        oracle.gather(host, blocks, np.arange(len(blocks)) * SHAPE.slot_bytes, ref,
                      SHAPE.layer_bytes)
        assert np.array_equal(_file_records(tmp_path / "daser.store", start, len(blocks)), ref)
    assert sorted(ipc.committed) == ["ka", "kb"]
    if stream.startswith("auto"):
        assert seen and all(x == (stream == "auto-side") for x in seen)
    w.shutdown()


@pytest.mark.parametrize("backend", ["native", "mmap"])
def test_load_round_trip_into_other_blocks(gpu, tmp_path, backend):
    print(f"case: connector load {backend}", flush=True)
    w, _ = _worker(tmp_path, io_backend=backend)
    caches = rand_caches(SHAPE, 16, "bf16", gpu, seed=32)
    named = _named(caches)
    w.register_kv_caches(named)
    _save(w, named, _store_reqs())
    w.shutdown()

    r, _ = _worker(tmp_path, io_backend=backend)
    fresh = [torch.zeros_like(c) for c in caches]
    r.register_kv_caches(_named(fresh))
    slot = SHAPE.slot_bytes
    meta = C.DaserConnectorMeta(reqs_to_load={
        "x": C.ReqLoadSpec("ka", 3, 3, [1, 12, 4], 3 * slot, 40),
        "y": C.ReqLoadSpec("kb", 10, 1, [0], 10 * slot, 16),
    })
    r.bind_connector_metadata(meta)
    r.start_load_kv(None)
    torch.cuda.synchronize()
    for c, f in zip(caches, fresh):
        assert torch.equal(f[:, [1, 12, 4, 0]], c[:, [5, 9, 2, 7]])
        untouched = [i for i in range(16) if i not in (1, 12, 4, 0)]
        assert not f[:, untouched].view(torch.int16).any()
    r.shutdown()


LLAMA31_SCALING = {"rope_type": "llama3", "factor": 8.0, "low_freq_factor": 1.0,
                   "high_freq_factor": 4.0, "original_max_position_embeddings": 8192}


@pytest.mark.parametrize("scaling", [None, LLAMA31_SCALING], ids=["plain", "llama3"])
def test_load_with_new_position_rerotates_k(gpu, tmp_path, scaling):
    """The rotation uses the model's frequencies; the scaled ones are pinned
    against transformers' own in the CPU tests of position.inv_freq_for."""
    print(f"case: connector load rerotate scaling={scaling}", flush=True)
    from daser_amd.position import inv_freq_for

    extra = {"rope_theta": 500000.0}
    if scaling:
        extra["rope_scaling"] = scaling
    w, _ = _worker(tmp_path, **extra)
    caches = rand_caches(SHAPE, 16, "bf16", gpu, seed=33)
    named = _named(caches)
    w.register_kv_caches(named)
    _save(w, named, _store_reqs())
    slot = SHAPE.slot_bytes
    recs = _file_records(tmp_path / "daser.store", 3, 3).copy()

    fresh = [torch.zeros_like(c) for c in caches]
    w2, _ = _worker(tmp_path, **extra)
    w2.register_kv_caches(_named(fresh))
    # stored at 100, placed at 4196: delta 4096; second request as stored
    meta = C.DaserConnectorMeta(reqs_to_load={
        "x": C.ReqLoadSpec("ka", 3, 3, [1, 12, 4], 3 * slot, 40, pos_offset=100, new_pos=4196),
        "y": C.ReqLoadSpec("kb", 10, 1, [0], 10 * slot, 16, pos_offset=5, new_pos=5),
    })
    w2.bind_connector_metadata(meta)
    w2.start_load_kv(None)
    torch.cuda.synchronize()
    ref = [np.zeros_like(to_bits_np(c, "bf16")) for c in caches]
    oracle.scatter_rerotate(ref, [1, 12, 4], np.arange(3) * slot, recs, SHAPE.layer_bytes,
                            dtype=oracle.BF16, rot_dim=64, style=oracle.NEOX,
                            stored_pos=np.full(3, 100), new_pos=np.full(3, 4196),
                            rotate=np.ones(3), theta=500000.0,
                            inv_freq=inv_freq_for(scaling, 64, 500000.0))
    for l, f in enumerate(fresh):
        got = to_bits_np(f, "bf16")
        assert np.array_equal(got[1][[1, 12, 4]], ref[l][1][[1, 12, 4]])
        ok, msg = oracle.rotation_within_tolerance(got[0][[1, 12, 4]], ref[l][0][[1, 12, 4]],
                                                   oracle.BF16)
        assert ok, msg
        assert torch.equal(f[:, 0], caches[l][:, 7])  # unchanged position: bit-exact
    w.shutdown()
    w2.shutdown()


def test_pinned_ring_device_round_trip(gpu, tmp_path):
    print("case: pinned ring", flush=True)
    path = str(tmp_path / "s.store")
    preallocate_store(path, 8 << 20)
    src = torch.randint(0, 256, (3_000_000,), dtype=torch.uint8, device=gpu)
    with PinnedRingIO(path, gpu, slot_bytes=1 << 18, n_slots=3) as io:
        io.write_from_device(src, 4096)
        dst = torch.zeros_like(src)
        io.read_into_device(dst, 4096)
        torch.cuda.synchronize()
    assert torch.equal(src, dst)


@pytest.mark.parametrize("uring,direct", [(True, False), (False, False), (True, True)])
def test_native_ring_device_round_trip(gpu, tmp_path, uring, direct):
    print(f"case: native ring uring={uring} direct={direct}", flush=True)
    path = str(tmp_path / "n.store")
    preallocate_store(path, 16 << 20)
    n = 5_000_001 if not direct else 5 << 20  # O_DIRECT: whole 4 KiB blocks
    src = torch.randint(0, 256, (n,), dtype=torch.uint8, device=gpu)
    with NativeRingIO(path, gpu, slot_bytes=1 << 20, n_slots=3, use_io_uring=uring,
                      direct=direct) as io:
        src.add_(1)  # producer-stream work the ring must wait for
        io.write_from_device(src, 65536)
        dst = torch.zeros_like(src)
        io.read_into_device(dst, 65536)
        dst.add_(0)  # consumer-stream work ordered after the copies
        torch.cuda.synchronize()
    assert torch.equal(src, dst)
    with open(path, "rb") as f:
        f.seek(65536)
        assert f.read(1000) == src[:1000].cpu().numpy().tobytes()


def test_missing_layer_saves_are_completed(gpu, tmp_path):
    """A layer whose save_kv_layer never ran is gathered in wait_for_save."""
    print("case: connector missing layer", flush=True)
    w, _ = _worker(tmp_path)
    caches = rand_caches(SHAPE, 16, "bf16", gpu, seed=34)
    named = _named(caches)
    w.register_kv_caches(named)
    w.bind_connector_metadata(C.DaserConnectorMeta(reqs_to_store=_store_reqs()))
    for i, (name, t) in enumerate(named.items()):
        if i != 1:
            w.save_kv_layer(name, t, None)
    w.wait_for_save()
    host = [to_bits_np(c, "bf16") for c in caches]
    ref = np.zeros(3 * SHAPE.slot_bytes, dtype=np.uint8)
    oracle.gather(host, [5, 9, 2], np.arange(3) * SHAPE.slot_bytes, ref, SHAPE.layer_bytes)
    assert np.array_equal(_file_records(tmp_path / "daser.store", 3, 3), ref)
    w.shutdown()


def test_batched_load_matches_single_batch(gpu, tmp_path):
    """Scattering per batch while later batches are read, with one reader
    ring or several in parallel, gives the same caches as one scatter after
    all reads, also when requests share a cached chunk (read once)."""
    print("case: batched load", flush=True)
    w, _ = _worker(tmp_path, rope_theta=500000.0)
    caches = rand_caches(SHAPE, 16, "bf16", gpu, seed=35)
    named = _named(caches)
    w.register_kv_caches(named)
    _save(w, named, _store_reqs())
    slot = SHAPE.slot_bytes
    reqs = {
        "x": C.ReqLoadSpec("ka", 3, 3, [1, 12, 4], 3 * slot, 40, pos_offset=0, new_pos=300),
        "y": C.ReqLoadSpec("kb", 10, 1, [0], 10 * slot, 16),
        # the same cached chunk again (read once, scattered twice), elsewhere
        "z": C.ReqLoadSpec("ka", 3, 3, [5, 6, 8], 3 * slot, 40, pos_offset=0, new_pos=9000),
        # part of it, as stored
        "w": C.ReqLoadSpec("ka", 0, 0, [9], 0, 16, segments=[C.LoadSegment(4, 1, 0)]),
    }
    plan = C.plan_load(reqs, slot)
    assert len(plan.reads) == 2 and plan.shared_records
    outs = []
    for batch, readers in ((1, 1), (1 << 30, 1), (1, 4), (1 << 30, 3)):
        fresh = [torch.zeros_like(c) for c in caches]
        p = C.KVDataPlane(str(tmp_path / "daser.store"), rope_theta=500000.0,
                          io_readers=readers, io_slot_bytes=4096, io_slots=2)
        p.register(_named(fresh))
        p.load(C.plan_load(reqs, slot), batch_bytes=batch)
        torch.cuda.synchronize()
        outs.append(fresh)
        p.close()
    for other in outs[1:]:
        for a, b in zip(outs[0], other):
            assert torch.equal(a, b)
    for l in range(SHAPE.num_layers):
        got = outs[0][l]
        assert torch.equal(got[:, 0], caches[l][:, 7])  # as stored
        assert torch.equal(got[:, 9], caches[l][:, 9])  # stored slot 4 = block 9
        # V of the shared chunk lands unchanged in both requests' blocks
        assert torch.equal(got[1][[1, 12, 4]], caches[l][1][[5, 9, 2]])
        assert torch.equal(got[1][[5, 6, 8]], caches[l][1][[5, 9, 2]])
        assert not torch.equal(got[0][[1, 12, 4]], got[0][[5, 6, 8]])  # two positions
    w.shutdown()


def test_save_without_layer_hooks_and_repeated_wait(gpu, tmp_path):
    """Under full graph replay no save_kv_layer runs: wait_for_save gathers
    every layer itself; a second wait_for_save in the step is a no-op."""
    print("case: connector save without hooks", flush=True)
    w, ipc = _worker(tmp_path)
    caches = rand_caches(SHAPE, 16, "bf16", gpu, seed=36)
    w.register_kv_caches(_named(caches))
    w.bind_connector_metadata(C.DaserConnectorMeta(reqs_to_store=_store_reqs()))
    w.wait_for_save()
    w.wait_for_save()
    host = [to_bits_np(c, "bf16") for c in caches]
    ref = np.zeros(3 * SHAPE.slot_bytes, dtype=np.uint8)
    oracle.gather(host, [5, 9, 2], np.arange(3) * SHAPE.slot_bytes, ref, SHAPE.layer_bytes)
    assert np.array_equal(_file_records(tmp_path / "daser.store", 3, 3), ref)
    assert sorted(ipc.committed) == ["ka", "kb"]  # committed once
    w.shutdown()


def test_unknown_layer_warns_and_others_still_save(gpu, tmp_path, caplog):
    """An unknown layer name in save_kv_layer is a warning and a skip, as in
    the reference (daser_connector.py:602-606); the known layers' records
    are still written and committed."""
    print("case: connector unknown layer", flush=True)
    w, ipc = _worker(tmp_path)
    caches = rand_caches(SHAPE, 16, "bf16", gpu, seed=37)
    named = _named(caches)
    w.register_kv_caches(named)
    w.bind_connector_metadata(C.DaserConnectorMeta(reqs_to_store=_store_reqs()))
    with caplog.at_level("WARNING"):
        w.save_kv_layer("model.layers.99.self_attn.attn", caches[0], None)
    assert any("unknown layer" in r.message for r in caplog.records)
    for name, t in named.items():
        w.save_kv_layer(name, t, None)
    w.wait_for_save()
    host = [to_bits_np(c, "bf16") for c in caches]
    ref = np.zeros(3 * SHAPE.slot_bytes, dtype=np.uint8)
    oracle.gather(host, [5, 9, 2], np.arange(3) * SHAPE.slot_bytes, ref, SHAPE.layer_bytes)
    assert np.array_equal(_file_records(tmp_path / "daser.store", 3, 3), ref)
    assert sorted(ipc.committed) == ["ka", "kb"]
    w.shutdown()


def test_fp8_load_rerotates_with_module_scales(gpu, tmp_path):
    """An e4m3 cache saved and reloaded at a new position through the
    connector: K is re-rotated with each layer's scale taken from the
    attention modules of the forward context, V and the unmoved request
    are bit-exact."""
    print("case: connector fp8 rerotate", flush=True)
    shape = KVShape(3, 2, 64, 16, 1)
    slot = shape.slot_bytes
    w, _ = _worker(tmp_path, rope_theta=500000.0)
    caches = rand_caches(shape, 16, "e4m3", gpu, seed=38, scale=40.0)
    named = _named(caches)
    w.register_kv_caches(named)
    _save(w, named, {"a": C.ReqStoreSpec("ka", 3, 3, [5, 9, 2], 3 * slot, 40),
                     "b": C.ReqStoreSpec("kb", 10, 1, [7], 10 * slot, 16)})
    recs = np.fromfile(tmp_path / "daser.store", dtype=np.uint8, count=3 * slot,
                       offset=3 * slot)
    scales = np.array([0.02, 0.05, 0.11], np.float32)
    fc = SimpleNamespace(no_compile_layers={
        n: SimpleNamespace(_k_scale=torch.tensor(float(v), device=gpu))
        for n, v in zip(named, scales)})
    fresh = [torch.zeros_like(c) for c in caches]
    w2, _ = _worker(tmp_path, rope_theta=500000.0)
    w2.register_kv_caches(_named(fresh))
    w2.bind_connector_metadata(C.DaserConnectorMeta(reqs_to_load={
        "x": C.ReqLoadSpec("ka", 3, 3, [1, 12, 4], 3 * slot, 40, pos_offset=100, new_pos=2148),
        "y": C.ReqLoadSpec("kb", 10, 1, [0], 10 * slot, 16, pos_offset=5, new_pos=5),
    }))
    w2.start_load_kv(fc)
    torch.cuda.synchronize()
    ref = [np.zeros_like(to_bits_np(c, "e4m3")) for c in caches]
    oracle.scatter_rerotate(ref, [1, 12, 4], np.arange(3) * slot, recs, shape.layer_bytes,
                            dtype=oracle.E4M3, rot_dim=64, style=oracle.NEOX,
                            stored_pos=np.full(3, 100), new_pos=np.full(3, 2148),
                            rotate=np.ones(3), theta=500000.0, k_scale=scales)
    for l, f in enumerate(fresh):
        got = to_bits_np(f, "e4m3")
        assert np.array_equal(got[1][[1, 12, 4]], ref[l][1][[1, 12, 4]])
        ok, msg = oracle.rotation_within_tolerance(got[0][[1, 12, 4]], ref[l][0][[1, 12, 4]],
                                                   oracle.E4M3)
        assert ok, f"layer {l}: {msg}"
        assert torch.equal(f[:, 0].view(torch.uint8), caches[l][:, 7].view(torch.uint8))
    w.shutdown()
    w2.shutdown()


@pytest.mark.parametrize("backend", ["native", "python", "mmap"])
def test_async_save_survives_immediate_block_reuse(gpu, tmp_path, backend):
    """async_save: wait_for_save returns before the file writes; the next
    step's KV writes to the same blocks (enqueued at once on the current
    stream) must not reach the records, and the chunks are committed once
    written (shutdown drains)."""
    print(f"case: connector async save {backend}", flush=True)
    w, ipc = _worker(tmp_path, async_save=True, io_backend=backend)
    caches = rand_caches(SHAPE, 16, "bf16", gpu, seed=39)
    host = [to_bits_np(c, "bf16") for c in caches]
    named = _named(caches)
    w.register_kv_caches(named)
    _save(w, named, _store_reqs())
    for c in caches:  # the blocks are reused right away
        c.fill_(3.0)
    second = {"c": C.ReqStoreSpec("kc", 20, 2, [5, 7], 20 * SHAPE.slot_bytes, 32)}
    _save(w, named, second)  # a second step queued behind the first
    w.shutdown()
    ref = np.zeros(3 * SHAPE.slot_bytes, dtype=np.uint8)
    oracle.gather(host, [5, 9, 2], np.arange(3) * SHAPE.slot_bytes, ref, SHAPE.layer_bytes)
    assert np.array_equal(_file_records(tmp_path / "daser.store", 3, 3), ref)
    filled = [to_bits_np(c, "bf16") for c in caches]
    ref2 = np.zeros(2 * SHAPE.slot_bytes, dtype=np.uint8)
    oracle.gather(filled, [5, 7], np.arange(2) * SHAPE.slot_bytes, ref2, SHAPE.layer_bytes)
    assert np.array_equal(_file_records(tmp_path / "daser.store", 20, 2), ref2)
    assert sorted(ipc.committed) == ["ka", "kb", "kc"]


class _FakeServer:
    """In-process stand-in of the DaseR server's chunk index: match_and_alloc
    (scheduler, sync) and commit_chunk (worker, async) over shared state, with
    the reply shapes the reference's IPC server uses."""

    def __init__(self, slot_bytes, block_tokens=16, stored_pos=None):
        # stored_pos: report committed chunks as stored at this position
        # (a position encoder that records where a chunk was prefilled)
        self.slot, self.bs, self.stored_pos = slot_bytes, block_tokens, stored_pos
        self.next_slot, self.pending, self.committed = 1, {}, {}

    def match_and_alloc(self, prefix, store_key, model_id):
        if store_key in self.committed:
            meta = dict(self.committed[store_key])
            if self.stored_pos is not None:
                meta["pos_offset"] = self.stored_pos
            return {"chunks": [meta], "alloc": None}
        n = len(prefix) // self.bs
        meta = {"chunk_key": store_key, "start_slot": self.next_slot, "num_slots": n,
                "file_offset": self.next_slot * self.slot, "token_count": n * self.bs,
                "pos_offset": 0}
        self.next_slot += n
        self.pending[store_key] = meta
        return {"chunks": [], "alloc": meta}

    async def commit_chunk(self, key):
        self.committed[key] = self.pending.pop(key)
        return {"ok": True}


def test_cold_then_warm_request_end_to_end(gpu, tmp_path):
    """The reference's integration check (tests/integration/test_vllm_e2e.py:
    177-181, cold == warm) at the connector level: a cold request is missed,
    allocated and saved by the worker; the same prompt later hits and its
    KV is loaded into other blocks bit-exactly; reported as stored at
    another position than the one it is placed at (0), it is re-rotated."""
    print("case: connector cold/warm end to end", flush=True)
    server = _FakeServer(SHAPE.slot_bytes)
    extra = dict(store_path=str(tmp_path / "daser.store"), io_slot_mb=0.03125, io_slots=3,
                 rope_theta=500000.0, block_tokens=16)
    cfg = SimpleNamespace(kv_transfer_config=SimpleNamespace(kv_connector_extra_config=extra))
    sched = C.DaserConnector(cfg, C.KVConnectorRole.SCHEDULER, ipc_client=server)
    worker = C.DaserConnector(cfg, C.KVConnectorRole.WORKER, ipc_async=server)
    caches = rand_caches(SHAPE, 16, "bf16", gpu, seed=41)
    named = _named(caches)
    worker.register_kv_caches(named)
    prompt = SimpleNamespace(request_id="cold", prompt_token_ids=list(range(1000, 1050)))

    def step(conn, req, blocks, hit, fc=None, save_named=None):
        conn_blocks = SimpleNamespace(blocks=[[SimpleNamespace(block_id=b) for b in blocks]])
        sched.update_state_after_alloc(req, conn_blocks, hit)
        meta = sched.build_connector_meta(
            SimpleNamespace(num_scheduled_tokens={req.request_id: len(req.prompt_token_ids)}))
        conn.bind_connector_metadata(meta)
        conn.start_load_kv(fc)
        for name, t in (save_named or {}).items():
            conn.save_kv_layer(name, t, None)
        conn.wait_for_save()
        conn.clear_connector_metadata()
        return meta

    assert sched.get_num_new_matched_tokens(prompt, 0) == (0, False)  # cold: miss
    meta = step(worker, prompt, [5, 9, 2, 11], 0, save_named=named)
    assert list(meta.reqs_to_store) == ["cold"] and not meta.reqs_to_load
    assert len(server.committed) == 1

    warm = SimpleNamespace(request_id="warm", prompt_token_ids=list(prompt.prompt_token_ids))
    assert sched.get_num_new_matched_tokens(warm, 0) == (48, False)  # 3 whole blocks
    fresh = [torch.zeros_like(c) for c in caches]
    w2 = C.DaserConnector(cfg, C.KVConnectorRole.WORKER, ipc_async=server)
    w2.register_kv_caches(_named(fresh))
    meta = step(w2, warm, [1, 12, 4, 7], 48)
    assert list(meta.reqs_to_load) == ["warm"]
    torch.cuda.synchronize()
    for l in range(SHAPE.num_layers):
        assert torch.equal(fresh[l][:, [1, 12, 4]], caches[l][:, [5, 9, 2]]), f"layer {l}"
        assert not fresh[l][:, 7].view(torch.int16).any()  # the uncached tail block

    # the same chunk reported as stored at position 700 and hit at 0: K
    # re-rotated by -700, V as stored
    server.stored_pos = 700
    moved = SimpleNamespace(request_id="moved", prompt_token_ids=list(prompt.prompt_token_ids))
    assert sched.get_num_new_matched_tokens(moved, 0) == (48, False)
    rot = [torch.zeros_like(c) for c in caches]
    w3 = C.DaserConnector(cfg, C.KVConnectorRole.WORKER, ipc_async=server)
    w3.register_kv_caches(_named(rot))
    step(w3, moved, [3, 6, 8, 0], 48)
    torch.cuda.synchronize()
    recs = _file_records(tmp_path / "daser.store", 1, 3).copy()
    ref = [np.zeros_like(to_bits_np(c, "bf16")) for c in caches]
    oracle.scatter_rerotate(ref, [3, 6, 8], np.arange(3) * SHAPE.slot_bytes, recs,
                            SHAPE.layer_bytes, dtype=oracle.BF16, rot_dim=64, style=oracle.NEOX,
                            stored_pos=np.full(3, 700), new_pos=np.zeros(3, np.int64),
                            rotate=np.ones(3), theta=500000.0)
    for l in range(SHAPE.num_layers):
        got = to_bits_np(rot[l], "bf16")
        assert torch.equal(rot[l][1][[3, 6, 8]], caches[l][1][[5, 9, 2]])
        ok, msg = oracle.rotation_within_tolerance(got[0][[3, 6, 8]], ref[l][0][[3, 6, 8]],
                                                   oracle.BF16)
        assert ok, f"layer {l}: {msg}"
    for w in (worker, w2, w3):
        w.shutdown()


def test_uncommitted_chunk_is_never_loaded(gpu, tmp_path):
    """With async_save the chunk is committed only after its records are in
    the file, so a lookup before that misses."""
    print("case: connector commit after write", flush=True)
    server = _FakeServer(SHAPE.slot_bytes)
    extra = dict(store_path=str(tmp_path / "daser.store"), io_slot_mb=0.03125, io_slots=3,
                 async_save=True)
    cfg = SimpleNamespace(kv_transfer_config=SimpleNamespace(kv_connector_extra_config=extra))
    sched = C.DaserConnector(cfg, C.KVConnectorRole.SCHEDULER, ipc_client=server)
    w = C.DaserConnector(cfg, C.KVConnectorRole.WORKER, ipc_async=server)
    caches = rand_caches(SHAPE, 16, "bf16", gpu, seed=42)
    w.register_kv_caches(_named(caches))
    req = SimpleNamespace(request_id="r", prompt_token_ids=list(range(32)))
    assert sched.get_num_new_matched_tokens(req, 0) == (0, False)
    assert server.pending and not server.committed  # allocated, not visible
    w.shutdown()


def test_load_rerotates_each_layer_with_its_rope(gpu, tmp_path):
    """rope_layers (local / global bases, a layer without RoPE): a moved
    chunk's K is rotated per layer with that layer's frequencies, and left
    as stored on the layer without RoPE."""
    print("case: connector per-layer rope", flush=True)
    rope = [{"rope_theta": 10000.0}, None, {"rope_theta": 1000000.0}]
    w, _ = _worker(tmp_path)
    caches = rand_caches(SHAPE, 16, "bf16", gpu, seed=43)
    named = _named(caches)
    w.register_kv_caches(named)
    _save(w, named, _store_reqs())
    slot = SHAPE.slot_bytes
    recs = _file_records(tmp_path / "daser.store", 3, 3).copy()
    fresh = [torch.zeros_like(c) for c in caches]
    w2, _ = _worker(tmp_path, rope_layers=rope)
    w2.register_kv_caches(_named(fresh))
    w2.bind_connector_metadata(C.DaserConnectorMeta(reqs_to_load={
        "x": C.ReqLoadSpec("ka", 3, 3, [1, 12, 4], 3 * slot, 40, pos_offset=100, new_pos=9000)}))
    w2.start_load_kv(None)
    torch.cuda.synchronize()
    for l, spec in enumerate(rope):
        ref = [np.zeros_like(to_bits_np(caches[l], "bf16"))]
        oracle.scatter_rerotate(ref, [1, 12, 4], np.arange(3) * slot, recs, SHAPE.layer_bytes,
                                dtype=oracle.BF16, rot_dim=64, style=oracle.NEOX,
                                stored_pos=np.full(3, 100), new_pos=np.full(3, 9000),
                                rotate=np.full(3, spec is not None),
                                theta=spec["rope_theta"] if spec else 1.0, layer0=l)
        got = to_bits_np(fresh[l], "bf16")
        assert np.array_equal(got[1][[1, 12, 4]], ref[0][1][[1, 12, 4]])
        if spec is None:
            assert np.array_equal(got[0][[1, 12, 4]], ref[0][0][[1, 12, 4]])
        ok, msg = oracle.rotation_within_tolerance(got[0][[1, 12, 4]], ref[0][0][[1, 12, 4]],
                                                   oracle.BF16)
        assert ok, f"layer {l}: {msg}"
    w.shutdown()
    w2.shutdown()


def test_flat_caches_save_and_rerotate_load(gpu, tmp_path):
    """vLLM's PagedAttention backend allocates (2, NB, block_size * H * D)
    caches with split-x K pages: saves write kv[:, b] bytes as the reference
    does, and a load at a new position re-rotates K in that layout, with the
    head geometry taken from cache_config and the hf_config."""
    print("case: connector 3-D caches", flush=True)
    hf = SimpleNamespace(hidden_size=128, num_attention_heads=2, rope_theta=500000.0)
    cfg = SimpleNamespace(
        kv_transfer_config=SimpleNamespace(kv_connector_extra_config=dict(
            store_path=str(tmp_path / "daser.store"), io_slot_mb=0.03125, io_slots=3)),
        model_config=SimpleNamespace(hf_config=hf),
        cache_config=SimpleNamespace(block_size=16, cache_dtype="auto"))
    caches = [c.reshape(2, 16, -1) for c in rand_caches(SHAPE, 16, "bf16", gpu, seed=35)]
    w = C.DaserConnector(cfg, C.KVConnectorRole.WORKER, ipc_async=FakeAsyncIPC())
    named = _named(caches)
    w.register_kv_caches(named)
    assert w._plane.table.layout.k_layout == "kx" and w._plane.table.layout.num_heads == 2
    _save(w, named, _store_reqs())
    slot = SHAPE.slot_bytes
    recs = _file_records(tmp_path / "daser.store", 3, 3).copy()
    want = np.concatenate([to_bits_np(c, "bf16")[:, b].reshape(-1).view(np.uint8)
                           for b in (5, 9, 2) for c in caches])
    assert np.array_equal(recs, want)  # bytes of kv[:, b], layer after layer

    fresh = [torch.zeros_like(c) for c in caches]
    w2 = C.DaserConnector(cfg, C.KVConnectorRole.WORKER, ipc_async=FakeAsyncIPC())
    w2.register_kv_caches(_named(fresh))
    w2.bind_connector_metadata(C.DaserConnectorMeta(reqs_to_load={
        "x": C.ReqLoadSpec("ka", 3, 3, [1, 12, 4], 3 * slot, 40, pos_offset=100,
                           new_pos=4196)}))
    w2.start_load_kv(None)
    torch.cuda.synchronize()
    to_nhd = lambda a: oracle.kx_to_nhd(a, 16, 2, 64)  # noqa: E731
    ref = [np.zeros((2, 16, 16, 2, 64), np.uint16) for _ in caches]
    recs_nhd = np.ascontiguousarray(to_nhd(recs.view(np.uint16).reshape(3, 3, 2, -1)))
    oracle.scatter_rerotate(ref, [1, 12, 4], np.arange(3) * slot,
                            recs_nhd.reshape(-1).view(np.uint8), SHAPE.layer_bytes,
                            dtype=oracle.BF16, rot_dim=64, style=oracle.NEOX,
                            stored_pos=np.full(3, 100), new_pos=np.full(3, 4196),
                            rotate=np.ones(3), theta=500000.0)
    for l, f in enumerate(fresh):
        got = to_nhd(to_bits_np(f, "bf16"))
        assert np.array_equal(got[1][[1, 12, 4]], ref[l][1][[1, 12, 4]])
        ok, msg = oracle.rotation_within_tolerance(got[0][[1, 12, 4]], ref[l][0][[1, 12, 4]],
                                                   oracle.BF16)
        assert ok, f"layer {l}: {msg}"
    w.shutdown()
    w2.shutdown()


def test_save_gathers_from_the_tensor_passed(gpu, tmp_path, caplog):
    """save_kv_layer copies from the kv_layer it receives, as the reference
    does (daser_connector.py:627-632): a tensor that is not the registered
    cache of that layer is gathered from, with one warning."""
    print("case: connector save from passed tensor", flush=True)
    w, _ = _worker(tmp_path)
    caches = rand_caches(SHAPE, 16, "bf16", gpu, seed=36)
    named = _named(caches)
    w.register_kv_caches(named)
    other = rand_caches(SHAPE, 16, "bf16", gpu, seed=37)
    passed = dict(named)
    passed["model.layers.1.self_attn.attn"] = other[1]
    with caplog.at_level("WARNING", logger="daser_amd.connector"):
        _save(w, passed, _store_reqs())
    assert "not the registered cache" in caplog.text
    host = [to_bits_np(c, "bf16") for c in (caches[0], other[1], caches[2])]
    ref = np.zeros(3 * SHAPE.slot_bytes, dtype=np.uint8)
    oracle.gather(host, [5, 9, 2], np.arange(3) * SHAPE.slot_bytes, ref, SHAPE.layer_bytes)
    assert np.array_equal(_file_records(tmp_path / "daser.store", 3, 3), ref)
    w.shutdown()


def test_head_major_caches_save_reference_records_and_load(gpu, tmp_path):
    """vLLM's HND layout (pages stored heads-first): the store file holds the
    same records as for token-major caches of the same values, and a load
    with a new position puts the same logical values back."""
    print("case: connector head-major caches", flush=True)

    def hnd(caches):
        out = []
        for c in caches:
            m = torch.empty((2, 16, SHAPE.num_heads, SHAPE.block_size, SHAPE.head_dim),
                            dtype=c.dtype, device=gpu)
            v = m.permute(0, 1, 3, 2, 4)
            v.copy_(c)
            out.append(v)
        return out

    caches = rand_caches(SHAPE, 16, "bf16", gpu, seed=38)
    w, _ = _worker(tmp_path, rope_theta=500000.0)
    named = _named(hnd(caches))
    w.register_kv_caches(named)
    assert w._plane.table.layout.k_layout == "hnd"
    _save(w, named, _store_reqs())
    host = [to_bits_np(c, "bf16") for c in caches]
    ref = np.zeros(3 * SHAPE.slot_bytes, dtype=np.uint8)
    oracle.gather(host, [5, 9, 2], np.arange(3) * SHAPE.slot_bytes, ref, SHAPE.layer_bytes)
    assert np.array_equal(_file_records(tmp_path / "daser.store", 3, 3), ref)

    slot = SHAPE.slot_bytes
    meta = C.DaserConnectorMeta(reqs_to_load={
        "x": C.ReqLoadSpec("ka", 3, 3, [1, 12, 4], 3 * slot, 40, pos_offset=100, new_pos=4196)})
    outs = []
    for layout in (hnd, lambda cs: cs):
        fresh = layout([torch.zeros_like(c) for c in caches])
        w2, _ = _worker(tmp_path, rope_theta=500000.0)
        w2.register_kv_caches(_named(fresh))
        w2.bind_connector_metadata(meta)
        w2.start_load_kv(None)
        torch.cuda.synchronize()
        outs.append([f.contiguous() for f in fresh])
        w2.shutdown()
    for a, b in zip(*outs):
        assert torch.equal(a.view(torch.int16), b.view(torch.int16))
    w.shutdown()


def random_load_reqs(rng, slot: int, n_slots: int, nb: int) -> dict:
    """Random load metadata of one step: 2-6 requests, flat or with 1-3
    segments; some segments inside ranges read earlier in the step; some
    blocks also loaded by the previous request; positions kept or moved."""
    reqs, used = {}, []
    for r in range(int(rng.integers(2, 7))):
        n_seg = int(rng.integers(1, 4))
        segs, boff = [], 0
        for _ in range(n_seg):
            n = int(rng.integers(1, 5))
            start = int(rng.integers(0, n_slots - n + 1))
            if used and rng.random() < 0.3:  # inside a range read earlier
                s0, n0 = used[int(rng.integers(0, len(used)))]
                n = min(n, n0)
                start = s0 + int(rng.integers(0, n0 - n + 1))
            used.append((start, n))
            pos = int(rng.integers(0, 5000)) if rng.random() < 0.5 else 0
            new = None if rng.random() < 0.3 else int(rng.integers(0, 20000))
            segs.append(C.LoadSegment(start, n, boff, pos, new))
            boff += n
        blocks = rng.choice(nb, boff, replace=False).tolist()
        if r and rng.random() < 0.5:  # a block an earlier request also loads
            prev = reqs[f"r{r - 1}"].block_ids
            b = prev[int(rng.integers(0, len(prev)))]
            if b not in blocks:
                blocks[int(rng.integers(0, boff))] = b
        s0 = segs[0]
        if n_seg == 1:
            reqs[f"r{r}"] = C.ReqLoadSpec(f"k{r}", s0.start_slot, s0.num_slots, blocks,
                                          s0.start_slot * slot, 16 * boff, s0.pos_offset,
                                          s0.new_pos)
        else:
            reqs[f"r{r}"] = C.ReqLoadSpec(f"k{r}", 0, 0, blocks, 0, 16 * boff, segments=segs)
    return reqs


def _head_major(caches):
    """The same logical caches stored heads-first (vLLM's HND layout)."""
    out = []
    for c in caches:
        _, nb, bs, h, d = c.shape
        m = torch.empty((2, nb, h, bs, d), dtype=c.dtype, device=c.device)
        v = m.permute(0, 1, 3, 2, 4)
        v.copy_(c)
        out.append(v)
    return out


def _to_split_x(c):
    """Token-major (2, NB, bs, H, D) caches as vLLM's 3-D PagedAttention caches
    (2, NB, bs * H * D), K and V pages both in the split-x order
    [H][D / X][bs][X] (a byte permutation of each page; only K's order
    matters to the kernels, V is moved as bytes)."""
    _, nb, bs, h, d = c.shape
    x = 16 // c.element_size()
    return (c.view(2, nb, bs, h, d // x, x).permute(0, 1, 3, 4, 2, 5).contiguous()
            .view(2, nb, bs * h * d))


def _from_split_x(c, bs, h, d):
    x = 16 // c.element_size()
    nb = c.shape[1]
    return c.view(2, nb, h, d // x, bs, x).permute(0, 1, 4, 2, 3, 5).reshape(2, nb, bs, h, d)


@pytest.mark.parametrize("seed", range(18))
def test_random_load_plans_match_the_sequential_oracle(gpu, tmp_path, seed):
    """Random loads of one step through the data plane: several requests,
    flat specs and multi-segment ones, segments that reuse ranges read
    earlier in the step, blocks that several loads target, positions
    changed or kept; read in one batch or many, by one ring or several;
    token-major, head-major or 3-D split-x caches, bf16 or e4m3 (per-layer
    K scales). The result equals the reference order applied page by page
    (request after request, segment after segment: the last load of a block
    wins), with each page re-rotated by the oracle."""
    layout = ("nhd", "hnd", "kx")[seed % 3]
    dt = ("bf16", "e4m3")[(seed // 3) % 2]
    print(f"case: random load plan seed={seed} {layout} {dt}", flush=True)
    rng = np.random.default_rng(100 + seed)
    shape = SHAPE if dt == "bf16" else KVShape(3, 2, 64, 16, 1)
    bs, h, d = shape.block_size, shape.num_heads, shape.head_dim
    slot, n_slots, nb, theta = shape.slot_bytes, 40, 48, 500000.0
    gen = torch.Generator().manual_seed(seed)
    if dt == "bf16":
        recs_t = torch.randn(n_slots * slot // 2, generator=gen).to(torch.bfloat16)
    else:
        recs_t = (torch.randn(n_slots * slot, generator=gen) * 40).to(torch.float8_e4m3fn)
    # the file holds records of the caches' own layout; the oracle works on
    # token-major pages, so split-x records are read through the inverse order
    file_recs = recs_t.view(torch.uint8).numpy()
    if layout == "kx":
        x = 16 // recs_t.element_size()
        recs_all = (recs_t.view(n_slots, shape.num_layers, 2, h, d // x, bs, x)
                    .permute(0, 1, 2, 5, 3, 4, 6).contiguous().view(torch.uint8).numpy()
                    .reshape(-1))
    else:
        recs_all = file_recs
    store = tmp_path / "daser.store"
    preallocate_store(str(store), n_slots * slot)
    with open(store, "r+b") as f:
        f.write(file_recs.tobytes())
    reqs = random_load_reqs(rng, slot, n_slots, nb)
    init = rand_caches(shape, nb, dt, gpu, seed=200 + seed, scale=1.0 if dt == "bf16" else 40.0)
    ref = [to_bits_np(c, dt) for c in init]
    scales = np.array([0.02, 0.05, 0.11], np.float32)
    kind = oracle.BF16 if dt == "bf16" else oracle.E4M3
    for spec in reqs.values():
        for sg in spec.resolved_segments():
            new = sg.pos_offset if sg.new_pos is None else sg.new_pos
            recs = np.ascontiguousarray(
                recs_all[sg.start_slot * slot:(sg.start_slot + sg.num_slots) * slot])
            oracle.scatter_rerotate(
                ref, spec.block_ids[sg.block_offset:sg.block_offset + sg.num_slots],
                np.arange(sg.num_slots) * slot, recs, shape.layer_bytes, dtype=kind,
                rot_dim=d, style=oracle.NEOX,
                stored_pos=np.full(sg.num_slots, sg.pos_offset),
                new_pos=np.full(sg.num_slots, new),
                rotate=np.full(sg.num_slots, new != sg.pos_offset), theta=theta,
                k_scale=scales if dt != "bf16" else None)
    for batch, readers in ((1, 1), (1 << 30, 3), (3 * slot, 2)):
        caches = [c.clone() for c in init]
        geometry = None
        if layout == "hnd":
            caches = _head_major(caches)
        elif layout == "kx":
            caches = [_to_split_x(c) for c in caches]
            geometry = {"block_size": bs, "head_dim": d}
        p = C.KVDataPlane(str(store), rope_theta=theta, io_readers=readers,
                          io_slot_bytes=4096, io_slots=2, cache_geometry=geometry,
                          k_scales=torch.from_numpy(scales).to(gpu) if dt != "bf16" else None)
        p.register(_named(caches))
        assert p.table.layout.k_layout == layout
        p.load(C.plan_load(reqs, slot), batch_bytes=batch)
        torch.cuda.synchronize()
        p.close()
        for l, c in enumerate(caches):
            c = _from_split_x(c, bs, h, d) if layout == "kx" else c
            got = to_bits_np(c.contiguous(), dt)
            assert np.array_equal(got[1], ref[l][1]), f"layer {l} V (batch {batch})"
            ok, msg = oracle.rotation_within_tolerance(got[0], ref[l][0], kind)
            assert ok, f"layer {l} K (batch {batch}): {msg}"


@pytest.mark.parametrize("seed", range(6))
def test_random_save_steps_match_the_oracle(gpu, tmp_path, seed):
    """Random save steps through the worker hooks: 1-5 requests of 1-6
    pages at random store slots (blocks may repeat across requests), the
    step saved per layer or deferred, blocking or with async_save, two steps
    in a row. Every request's records in the file equal the oracle's gather
    of its blocks, and every chunk is committed."""
    print(f"case: random save steps seed={seed}", flush=True)
    rng = np.random.default_rng(300 + seed)
    mode = ("per_layer", "deferred")[seed % 2]
    async_save = seed % 3 == 0
    nb, slot = 40, SHAPE.slot_bytes
    w, ipc = _worker(tmp_path, save_mode=mode, async_save=async_save)
    caches = rand_caches(SHAPE, nb, "bf16", gpu, seed=400 + seed)
    named = _named(caches)
    w.register_kv_caches(named)
    host = [to_bits_np(c, "bf16") for c in caches]
    expect, free = {}, list(rng.permutation(60))
    for step in range(2):
        reqs = {}
        for r in range(int(rng.integers(1, 6))):
            n = int(rng.integers(1, 7))
            start = int(free.pop()) * 8  # disjoint 8-slot ranges of the store
            blocks = rng.choice(nb, n, replace=False).tolist()
            key = f"k{step}_{r}"
            reqs[f"s{step}_{r}"] = C.ReqStoreSpec(key, start, n, blocks, start * slot, 16 * n)
            expect[key] = (start, blocks)
        _save(w, named, reqs)
    w.shutdown()  # drains async writes
    for key, (start, blocks) in expect.items():
        ref = np.zeros(len(blocks) * slot, dtype=np.uint8)
        oracle.gather(host, blocks, np.arange(len(blocks)) * slot, ref, SHAPE.layer_bytes)
        got = _file_records(tmp_path / "daser.store", start, len(blocks))
        assert np.array_equal(got, ref), key
    assert sorted(ipc.committed) == sorted(expect)


def test_store_path_per_rank(gpu, tmp_path, monkeypatch):
    """A store_path with {rank}: the worker of tensor-parallel rank 1 writes
    its records to its own file, in the reference's layout."""
    print("case: connector per-rank store file", flush=True)
    monkeypatch.setenv("LOCAL_RANK", "1")
    cfg = SimpleNamespace(kv_transfer_config=SimpleNamespace(kv_connector_extra_config=dict(
        store_path=str(tmp_path / "daser.{rank}.store"), io_slot_mb=0.03125, io_slots=3)))
    w = C.DaserConnector(cfg, C.KVConnectorRole.WORKER, ipc_async=FakeAsyncIPC())
    caches = rand_caches(SHAPE, 16, "bf16", gpu, seed=44)
    named = _named(caches)
    w.register_kv_caches(named)
    _save(w, named, _store_reqs())
    w.shutdown()
    assert (tmp_path / "daser.1.store").exists() and not (tmp_path / "daser.{rank}.store").exists()
    host = [to_bits_np(c, "bf16") for c in caches]
    ref = np.zeros(3 * SHAPE.slot_bytes, dtype=np.uint8)
    oracle.gather(host, [5, 9, 2], np.arange(3) * SHAPE.slot_bytes, ref, SHAPE.layer_bytes)
    with open(tmp_path / "daser.1.store", "rb") as f:
        f.seek(3 * SHAPE.slot_bytes)
        assert np.array_equal(np.frombuffer(f.read(ref.size), np.uint8), ref)
