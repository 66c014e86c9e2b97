"""Load positions produced by the scheduler, end to end on the GPU: the
server's index (daser_amd.retrieval) answers the scheduler, which places each
chunk in the prompt; the worker re-rotates K from the chunk's stored
position to that place. Checked against oracle.scatter_rerotate on the
records in the store file."""

from __future__ import annotations

import asyncio

import numpy as np
import pytest
import torch

from daser_amd import connector as C
from daser_amd.retrieval import ChunkAssemblyIndex, IncrementalPrefixIndex, chunk_key
from oracle import oracle
from tests.helpers import rand_caches, to_bits_np
from tests.test_connector_gpu import SHAPE, _file_records, _named, _save, _worker
from tests.test_retrieval import ServerWithIndex, meta_for, _schedule, _scheduler

pytestmark = pytest.mark.gpu

THETA = 500000.0
NB = 128
BS = SHAPE.block_size


def _store_chunks(tmp_path, gpu, chunks, seed):
    """Saves each (tokens, start_slot) chunk's pages from seeded source
    caches through the worker hooks; returns the worker (still open)."""
    w, _ = _worker(tmp_path, rope_theta=THETA)
    src = rand_caches(SHAPE, NB, "bf16", gpu, seed=seed)
    named = _named(src)
    w.register_kv_caches(named)
    rng = np.random.default_rng(seed)
    blocks = rng.permutation(NB).tolist()
    reqs, used = {}, 0
    for i, (toks, start) in enumerate(chunks):
        n = -(-len(toks) // BS)
        reqs[f"s{i}"] = C.ReqStoreSpec(chunk_key(toks), start, n, blocks[used:used + n],
                                       start * SHAPE.slot_bytes, len(toks))
        used += n
    _save(w, named, reqs)
    return w


def _load_and_check(tmp_path, gpu, spec, expect):
    """Runs the worker load of ``spec`` into fresh caches and compares every
    loaded page with the oracle. expect: (start_slot, n_pages, block_offset,
    stored_pos, new_pos) per segment."""
    w2, _ = _worker(tmp_path, rope_theta=THETA)
    fresh = rand_caches(SHAPE, NB, "bf16", gpu, seed=99)
    w2.register_kv_caches(_named(fresh))
    ref = [to_bits_np(c, "bf16") for c in fresh]
    w2.bind_connector_metadata(C.DaserConnectorMeta(reqs_to_load={"r": spec}))
    w2.start_load_kv(None)
    torch.cuda.synchronize()
    slot = SHAPE.slot_bytes
    for start, n, boff, stored, new in expect:
        recs = _file_records(tmp_path / "daser.store", start, n).copy()
        dst = spec.block_ids[boff:boff + n]
        oracle.scatter_rerotate(ref, dst, np.arange(n) * slot, recs, SHAPE.layer_bytes,
                                dtype=oracle.BF16, rot_dim=SHAPE.head_dim, style=oracle.NEOX,
                                stored_pos=np.full(n, stored), new_pos=np.full(n, new),
                                rotate=np.full(n, new != stored), theta=THETA)
    for l, f in enumerate(fresh):
        got = to_bits_np(f, "bf16")
        assert np.array_equal(got[1], ref[l][1]), f"layer {l}: V"
        ok, msg = oracle.rotation_within_tolerance(got[0], ref[l][0], oracle.BF16)
        assert ok, f"layer {l}: {msg}"
    w2.shutdown()
    return fresh


def test_chunk_stored_at_3000_prefix_hit_at_0_is_rotated_back(gpu, tmp_path):
    print("case: positions prefix hit stored 3000 -> 0", flush=True)
    rng = np.random.default_rng(10)
    toks = rng.integers(0, 30000, size=160).tolist()
    w = _store_chunks(tmp_path, gpu, [(toks, 12)], seed=41)
    idx = IncrementalPrefixIndex(BS)
    asyncio.run(idx.insert(meta_for(toks, 12, model_id="m", pos_offset=3000)))
    n, spec = _schedule(_scheduler(ServerWithIndex(idx, SHAPE.slot_bytes)), "r",
                        toks + [7, 7, 7], 12, rng.permutation(NB))
    assert n == 160 and (spec.pos_offset, spec.new_pos) == (3000, 0)
    fresh = _load_and_check(tmp_path, gpu, spec, [(12, 10, 0, 3000, 0)])
    # K really moved: a stored-at-0 chunk would load bit-exact
    recs = _file_records(tmp_path / "daser.store", 12, 1).view(np.uint16)
    k0 = to_bits_np(fresh[0], "bf16")[0][spec.block_ids[0]].reshape(-1)
    assert (k0 != recs[:k0.size]).mean() > 0.5
    w.shutdown()


def test_two_chunks_assembled_at_0_and_528(gpu, tmp_path):
    print("case: positions two chunks at 0 and 528", flush=True)
    rng = np.random.default_rng(11)
    a = rng.integers(0, 30000, size=528).tolist()  # 33 pages, stored at 0
    b = rng.integers(0, 30000, size=256).tolist()  # 16 pages, stored at 0
    w = _store_chunks(tmp_path, gpu, [(a, 40), (b, 200)], seed=42)
    idx = ChunkAssemblyIndex(BS)
    for toks, start in ((a, 40), (b, 200)):
        asyncio.run(idx.insert(meta_for(toks, start, model_id="m", pos_offset=0)))
    n, spec = _schedule(_scheduler(ServerWithIndex(idx, SHAPE.slot_bytes)), "r",
                        a + b + [3] * 30, 60, rng.permutation(NB))
    assert n == 784 and len(spec.segments) == 2
    _load_and_check(tmp_path, gpu, spec, [(40, 33, 0, 0, 0), (200, 16, 33, 0, 528)])
    w.shutdown()


def test_vllm_prefix_hit_keeps_its_blocks(gpu, tmp_path):
    """vLLM computed the first 80 tokens itself (its local prefix cache):
    the load leaves those 5 blocks alone and fills the rest, the second chunk
    re-rotated from its stored position 1000 to 528."""
    print("case: positions num_computed_tokens=80, chunks at 0 and 528", flush=True)
    rng = np.random.default_rng(12)
    a = rng.integers(0, 30000, size=528).tolist()
    b = rng.integers(0, 30000, size=256).tolist()
    w = _store_chunks(tmp_path, gpu, [(a, 40), (b, 200)], seed=43)
    idx = ChunkAssemblyIndex(BS)
    asyncio.run(idx.insert(meta_for(a, 40, model_id="m", pos_offset=0)))
    asyncio.run(idx.insert(meta_for(b, 200, model_id="m", pos_offset=1000)))
    blocks = rng.permutation(NB)
    n, spec = _schedule(_scheduler(ServerWithIndex(idx, SHAPE.slot_bytes)), "r",
                        a + b + [3] * 30, 60, blocks, computed=80)
    assert n == 784 - 80 and spec.block_ids == blocks[5:49].tolist()
    # _load_and_check also holds every page it does not load (blocks[:5]) to
    # its old bytes
    _load_and_check(tmp_path, gpu, spec, [(45, 28, 0, 80, 80), (200, 16, 28, 1000, 528)])
    w.shutdown()


def test_duplicate_destination_blocks_keep_the_last_load(gpu, tmp_path):
    """Loads of one step that target the same block leave the last one's
    bytes, as the reference's sequential copies do (daser_connector.py:
    536-551): x loads chunk A into [3, 9], y chunk B into [9, 4], z chunk A
    again into [4, 11] (z reuses x's read, so without care it would be
    scattered before y). Checked against the oracle's sequential scatter of
    x, y, z."""
    print("case: positions duplicate destination keeps the last load", flush=True)
    rng = np.random.default_rng(12)
    ta = rng.integers(0, 30000, size=32).tolist()
    tb = rng.integers(0, 30000, size=32).tolist()
    w = _store_chunks(tmp_path, gpu, [(ta, 5), (tb, 20)], seed=43)
    w.shutdown()
    w2, _ = _worker(tmp_path)
    fresh = rand_caches(SHAPE, NB, "bf16", gpu, seed=1)
    ref = [to_bits_np(c, "bf16") for c in fresh]
    w2.register_kv_caches(_named(fresh))
    slot = SHAPE.slot_bytes
    loads = {"x": (5, [3, 9]), "y": (20, [9, 4]), "z": (5, [4, 11])}
    w2.bind_connector_metadata(C.DaserConnectorMeta(reqs_to_load={
        r: C.ReqLoadSpec("k" + r, start, 2, blocks, start * slot, 32)
        for r, (start, blocks) in loads.items()}))
    w2.start_load_kv(None)
    torch.cuda.synchronize()
    for start, blocks in loads.values():
        recs = _file_records(tmp_path / "daser.store", start, 2).copy()
        oracle.scatter(ref, blocks, np.arange(2) * slot, recs, SHAPE.layer_bytes)
    for l, f in enumerate(fresh):
        assert np.array_equal(to_bits_np(f, "bf16"), ref[l]), f"layer {l}"
    w2.shutdown()
