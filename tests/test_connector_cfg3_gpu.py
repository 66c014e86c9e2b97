"""The connector's whole load path at the RAG chunk-reuse workload's shape
(Llama-3-8B KV: 32 layers, 8 KV heads, head_dim 128, block_size 16):

  1. 16 separately prefilled 512-token chunks are saved, four per step,
     through save_kv_layer / wait_for_save into the store file
     (reference daser/connector/daser_connector.py:574-684);
  2. they are inserted into ChunkAssemblyIndex (the server's index);
  3. three RAG prompts of 10 chunks plus a question go through
     get_num_new_matched_tokens -> update_state_after_alloc ->
     build_connector_meta, which place each chunk at its prompt position;
  4. one start_load_kv reads the records and scatters them into vLLM's
     blocks, re-rotating K from each chunk's stored position
     (reference :455-558 for the copy; the rotation is this path's own).

64 loaded pages (all layers) are then checked against
oracle.scatter_rerotate on the store file's records: V bit-exact, K within
the rotation tolerance (1 ulp, a 2^-18 row-relative allowance for
cancellation); pages of the cache that no load targets keep their bytes.
"""

from __future__ import annotations

import asyncio
from types import SimpleNamespace

import numpy as np
import pytest
import torch

from daser_amd import connector as C
from daser_amd.retrieval import ChunkAssemblyIndex, ChunkMeta, chunk_key
from daser_amd.workloads import LLAMA3_8B, LLAMA3_8B_FP8
from oracle import oracle
from tests.helpers import BITS_T, ORC_DT, TORCH_DT, to_bits_np

pytestmark = pytest.mark.gpu

THETA = 500000.0
BS = 16
CHUNK = 512                 # tokens per cached chunk
PAGES = CHUNK // BS         # 32
N_CHUNKS = 16
PER_PROMPT = 10
N_PROMPTS = 3
NB_SRC = N_CHUNKS * PAGES + 16
NB = 1024                   # vLLM's block pool of the loading worker
SAMPLE = 64


class _Commits:
    def __init__(self):
        self.committed = []

    async def commit_chunk(self, key):
        self.committed.append(key)
        return {"ok": True}


class _IndexServer:
    """match_and_alloc answered from a ChunkAssemblyIndex (the server's
    lookup); nothing is allocated, as for a prompt whose chunks are cached."""

    def __init__(self, index, slot_bytes):
        self.index, self.slot = index, slot_bytes

    def match_and_alloc(self, tokens, store_key, model_id):
        found = asyncio.run(self.index.lookup(tokens, model_id))
        return {"chunks": [{"chunk_key": m.chunk_key, "start_slot": m.start_slot,
                            "num_slots": m.num_slots, "token_count": m.token_count,
                            "pos_offset": m.pos_offset, "file_offset": m.start_slot * self.slot}
                           for m in found], "alloc": None}


def _caches(shape, nb, dt, device, seed):
    """(2, nb, bs, H, D) per layer, ~N(0, 1), drawn on the device."""
    g = torch.Generator(device=device).manual_seed(seed)
    return [torch.randn((2, nb, shape.block_size, shape.num_heads, shape.head_dim),
                        generator=g, device=device).to(TORCH_DT[dt])
            for _ in range(shape.num_layers)]


def _named(caches):
    return {f"model.layers.{i}.self_attn.attn": c for i, c in enumerate(caches)}


def _cfg(tmp_path, dt, **extra):
    cache = SimpleNamespace(block_size=BS, cache_dtype="fp8" if dt == "e4m3" else "auto")
    return SimpleNamespace(
        cache_config=cache,
        kv_transfer_config=SimpleNamespace(kv_connector_extra_config=dict(
            store_path=str(tmp_path / "daser.store"), rope_theta=THETA, block_tokens=BS,
            model_id="m", allow_chunk_assembly=True, **extra)))


def _records(path, slot_bytes, slots):
    """The store file's records of the given slots, one after another."""
    out = np.empty(len(slots) * slot_bytes, np.uint8)
    with open(path, "rb") as f:
        for i, s in enumerate(slots):
            f.seek(int(s) * slot_bytes)
            out[i * slot_bytes:(i + 1) * slot_bytes] = np.frombuffer(f.read(slot_bytes), np.uint8)
    return out


@pytest.mark.parametrize("dt", ["bf16", "e4m3"])
def test_rag_assembly_at_llama3_8b_shape(gpu, tmp_path, dt):
    print(f"case: connector cfg3 shape rag assembly {dt}", flush=True)
    shape = LLAMA3_8B if dt == "bf16" else LLAMA3_8B_FP8
    slot = shape.slot_bytes
    rng = np.random.default_rng(2024 if dt == "bf16" else 2025)
    cfg = _cfg(tmp_path, dt)
    # per-layer K scales of the fp8 cache, as vLLM keeps them on the
    # attention modules (forward_context.no_compile_layers[name]._k_scale)
    scales = (0.5 + rng.random(shape.num_layers)).astype(np.float32)
    names = list(_named(range(shape.num_layers)))
    fc = SimpleNamespace(no_compile_layers={
        n: SimpleNamespace(_k_scale=torch.tensor(float(s), device=gpu))
        for n, s in zip(names, scales)})

    # 1. save: 16 chunks of 32 pages, four chunks per step; each chunk is
    # stored at position 0 (its own prefill) but four of them at another one
    saver = C.DaserConnector(cfg, C.KVConnectorRole.WORKER, ipc_async=_Commits())
    src = _caches(shape, NB_SRC, dt, gpu, seed=7)
    named_src = _named(src)
    saver.register_kv_caches(named_src)
    assert saver._slot_size == slot
    docs = [rng.integers(0, 120000, CHUNK).tolist() for _ in range(N_CHUNKS)]
    stored_pos = np.zeros(N_CHUNKS, np.int64)
    stored_pos[rng.choice(N_CHUNKS, 4, replace=False)] = rng.integers(1, 32768, 4)
    start_slots = rng.permutation(N_CHUNKS) * PAGES + 8  # scattered through the file
    src_blocks = rng.permutation(NB_SRC)[:N_CHUNKS * PAGES].reshape(N_CHUNKS, PAGES)
    for step in range(N_CHUNKS // 4):
        reqs = {}
        for c in range(step * 4, step * 4 + 4):
            reqs[f"p{c}"] = C.ReqStoreSpec(chunk_key(docs[c]), int(start_slots[c]), PAGES,
                                           src_blocks[c].tolist(), int(start_slots[c]) * slot,
                                           CHUNK)
        saver.bind_connector_metadata(C.DaserConnectorMeta(reqs_to_store=reqs))
        for name, t in named_src.items():
            saver.save_kv_layer(name, t, None)
        saver.wait_for_save()
        saver.clear_connector_metadata()
    assert sorted(saver._ipc_async.committed) == sorted(chunk_key(d) for d in docs)
    saver.shutdown()
    # the saved records are the source pages (gather parity, sampled)
    probe = rng.integers(0, N_CHUNKS, 2)
    for c in probe:
        got = _records(tmp_path / "daser.store", slot, [int(start_slots[c]) + 5])
        host = [to_bits_np(x[:, [int(src_blocks[c][5])]], dt) for x in src]
        ref = np.zeros(slot, np.uint8)
        oracle.gather(host, [0], [0], ref, shape.layer_bytes)
        assert np.array_equal(got, ref), f"saved record of chunk {c}"
    del src, named_src
    torch.cuda.empty_cache()

    # 2. the server's index
    idx = ChunkAssemblyIndex(BS)
    for c in range(N_CHUNKS):
        asyncio.run(idx.insert(ChunkMeta(chunk_key(docs[c]), int(start_slots[c]), PAGES, CHUNK,
                                         int(stored_pos[c]), "m")))

    # 3. the scheduler places 10 chunks per prompt; vLLM's blocks are a
    # random draw from the pool, disjoint between prompts
    sched = C.DaserConnector(cfg, C.KVConnectorRole.SCHEDULER,
                             ipc_client=_IndexServer(idx, slot))
    pool = rng.permutation(NB)
    need = PER_PROMPT * PAGES + 2
    meta_all = C.DaserConnectorMeta()
    picks = []
    for r in range(N_PROMPTS):
        pick = rng.choice(N_CHUNKS, PER_PROMPT, replace=False)
        picks.append(pick)
        prompt = [t for c in pick for t in docs[c]] + rng.integers(0, 120000, 20).tolist()
        req = SimpleNamespace(request_id=f"rag{r}", prompt_token_ids=prompt)
        n, _ = sched.get_num_new_matched_tokens(req, 0)
        assert n == PER_PROMPT * CHUNK
        mine = pool[r * need:(r + 1) * need].tolist()
        sched.update_state_after_alloc(
            req, SimpleNamespace(blocks=[[SimpleNamespace(block_id=b) for b in mine]]), n)
        meta = sched.build_connector_meta(
            SimpleNamespace(num_scheduled_tokens={req.request_id: len(prompt)}))
        spec = meta.reqs_to_load[req.request_id]
        assert [(s.start_slot, s.num_slots, s.block_offset, s.pos_offset, s.new_pos)
                for s in spec.segments] == \
            [(int(start_slots[c]), PAGES, i * PAGES, int(stored_pos[c]), i * CHUNK)
             for i, c in enumerate(pick)]
        meta_all.reqs_to_load.update(meta.reqs_to_load)

    # 4. one load for the three prompts
    loader = C.DaserConnector(cfg, C.KVConnectorRole.WORKER, ipc_async=_Commits())
    dst = _caches(shape, NB, dt, gpu, seed=8)
    loader.register_kv_caches(_named(dst))
    untouched = pool[N_PROMPTS * need:][:8]
    before = [to_bits_np(x[:, untouched], dt) for x in dst]
    loader.bind_connector_metadata(meta_all)
    loader.start_load_kv(fc)
    torch.cuda.synchronize()
    loader.clear_connector_metadata()
    loader.shutdown()

    # every loaded page: (block, store slot, stored position, new position)
    pages = []
    for r, pick in enumerate(picks):
        blocks = pool[r * need:(r + 1) * need]
        for i, c in enumerate(pick):
            for j in range(PAGES):
                pages.append((int(blocks[i * PAGES + j]), int(start_slots[c]) + j,
                              int(stored_pos[c]), i * CHUNK))
    pages = np.asarray(pages, np.int64)
    sel = pages[rng.choice(len(pages), SAMPLE, replace=False)]
    recs = _records(tmp_path / "daser.store", slot, sel[:, 1])
    ref = [np.zeros((2, SAMPLE, BS, shape.num_heads, shape.head_dim), to_bits_np(
        dst[0][:, :1], dt).dtype) for _ in range(shape.num_layers)]
    oracle.scatter_rerotate(ref, np.arange(SAMPLE), np.arange(SAMPLE) * slot, recs,
                            shape.layer_bytes, dtype=ORC_DT[dt], rot_dim=shape.head_dim,
                            style=oracle.NEOX, stored_pos=sel[:, 2], new_pos=sel[:, 3],
                            rotate=sel[:, 2] != sel[:, 3], theta=THETA,
                            k_scale=scales if dt == "e4m3" else None)
    moved = sel[:, 2] != sel[:, 3]
    assert moved.sum() >= SAMPLE // 2, "most sampled pages are re-rotated"
    for l in range(shape.num_layers):
        got = to_bits_np(dst[l][:, sel[:, 0]], dt)
        assert np.array_equal(got[1], ref[l][1]), f"layer {l}: V"
        assert np.array_equal(got[0][~moved], ref[l][0][~moved]), f"layer {l}: unmoved K"
        ok, msg = oracle.rotation_within_tolerance(got[0], ref[l][0], ORC_DT[dt])
        assert ok, f"layer {l}: {msg}"
        assert np.array_equal(to_bits_np(dst[l][:, untouched], dt), before[l]), \
            f"layer {l}: a page no load targets changed"
