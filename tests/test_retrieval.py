"""Retrieval indexes (daser_amd.retrieval) and the scheduler's placement of
the chunks they return: the reference's longest-prefix lookup in one hashing
pass, multi-chunk assembly of RAG prompts, and the load positions the
scheduler derives from it (no GPU)."""

from __future__ import annotations

import asyncio
import math
from types import SimpleNamespace

import numpy as np
import pytest

from daser_amd import connector as C
from daser_amd.retrieval import ChunkAssemblyIndex, ChunkMeta, IncrementalPrefixIndex, chunk_key

BS = 16
SLOT = 4096


def run(coro):
    return asyncio.run(coro)


def reference_scan(index: dict, tokens: list[int], model_id: str, bs: int = BS):
    """The reference's PrefixHashIndex.lookup (daser/retrieval/prefix.py:
    49-72): hash every block-aligned prefix from scratch, longest first."""
    n = len(tokens) // bs * bs
    while n >= bs:
        meta = index.get(chunk_key(tokens[:n]))
        if meta is not None and meta.model_id == model_id:
            return [meta]
        n -= bs
    return []


def meta_for(tokens, start_slot, model_id="m", pos_offset=0):
    return ChunkMeta(chunk_key(tokens), start_slot, math.ceil(len(tokens) / BS), len(tokens),
                     pos_offset, model_id)


def test_chunk_key_is_the_reference_hash():
    assert chunk_key([1, 2, 3]) == C.hash_tokens([1, 2, 3])
    assert chunk_key(np.arange(40, dtype=np.int64)) == C.hash_tokens(list(range(40)))


def test_incremental_prefix_index_equals_reference_scan():
    rng = np.random.default_rng(0)
    for trial in range(30):
        base = rng.integers(0, 50000, size=int(rng.integers(0, 700))).tolist()
        idx = IncrementalPrefixIndex(BS)
        stored = {}
        for k in range(int(rng.integers(0, 6))):
            n = int(rng.integers(1, len(base) // BS + 2)) * BS
            toks = base[:n] if rng.random() < 0.7 else rng.integers(0, 9, n).tolist()
            m = meta_for(toks, k, model_id="m" if rng.random() < 0.8 else "other")
            run(idx.insert(m))
            stored[m.chunk_key] = m
        if stored and rng.random() < 0.3:
            key = next(iter(stored))
            run(idx.remove(key))
            del stored[key]
        query = base + rng.integers(0, 50000, size=int(rng.integers(0, 40))).tolist()
        for model in ("m", "other"):
            assert run(idx.lookup(query, model)) == reference_scan(stored, query, model), trial
    run(IncrementalPrefixIndex(BS).remove("absent"))  # unknown keys are ignored


def _docs(rng, n_docs=3, chunk_tokens=64):
    """Documents split into fixed chunks, as the reference service's
    chunker does (daser/service/chunker.py), each a cached chunk."""
    docs = [rng.integers(0, 30000, size=chunk_tokens * int(rng.integers(1, 4))).tolist()
            for _ in range(n_docs)]
    chunks = [d[i:i + chunk_tokens] for d in docs for i in range(0, len(d), chunk_tokens)]
    return docs, chunks


def test_assembly_index_tiles_a_rag_prompt():
    rng = np.random.default_rng(1)
    docs, chunks = _docs(rng)
    idx = ChunkAssemblyIndex(BS)
    for i, c in enumerate(chunks):
        run(idx.insert(meta_for(c, 100 + 10 * i)))
    question = rng.integers(0, 30000, size=37).tolist()
    prompt = docs[2] + docs[0] + question
    got = run(idx.lookup(prompt, "m"))
    want = [chunk_key(d[i:i + 64]) for d in (docs[2], docs[0]) for i in range(0, len(d), 64)]
    assert [m.chunk_key for m in got] == want
    # the first reply chunk is the reference's longest-prefix hit
    assert got[:1] == reference_scan({m.chunk_key: m for m in got}, prompt, "m")
    # another model's chunks are invisible; a gap stops the tiling
    assert run(idx.lookup(prompt, "other")) == []
    gap = docs[1][:64] + question[:16] + docs[0]
    assert [m.chunk_key for m in run(idx.lookup(gap, "m"))] == [chunk_key(docs[1][:64])]
    # a longer cached chunk (a whole earlier prompt) wins over its pieces
    whole = meta_for(docs[2] + docs[0][:64], 900)
    run(idx.insert(whole))
    got = run(idx.lookup(prompt, "m"))
    assert got[0] is whole and len(got) == 1 + len(docs[0]) // 64 - 1
    idx2 = ChunkAssemblyIndex(BS, max_chunks=2)
    for i, c in enumerate(chunks):
        run(idx2.insert(meta_for(c, i)))
    assert len(run(idx2.lookup(prompt, "m"))) == 2


class ServerWithIndex:
    """The reference IPC server's match_and_alloc reply
    (daser/server/ipc_server.py:256-291) over a RetrievalIndex."""

    def __init__(self, index, slot_bytes=SLOT):
        self.index, self.slot, self.calls = index, slot_bytes, []

    def match_and_alloc(self, tokens, chunk_key_, model_id):
        self.calls.append(len(tokens))
        chunks = asyncio.run(self.index.lookup(tokens, model_id))
        return {"chunks": [{"chunk_key": m.chunk_key, "start_slot": m.start_slot,
                            "num_slots": m.num_slots, "token_count": m.token_count,
                            "pos_offset": m.pos_offset, "model_id": m.model_id,
                            "file_offset": m.start_slot * self.slot} for m in chunks],
                "alloc": None}


def _scheduler(server, assemble=True):
    cfg = SimpleNamespace(kv_transfer_config=SimpleNamespace(
        kv_connector_extra_config={"block_tokens": BS, "model_id": "m",
                                   "allow_chunk_assembly": assemble}))
    return C.DaserConnector(cfg, C.KVConnectorRole.SCHEDULER, ipc_client=server)


def _schedule(conn, rid, prompt, n_blocks, block_ids=None, computed=0):
    """One request through the scheduler hooks; vLLM's blocks are
    ``block_ids`` (default 1000, 1001, ...), of which the first
    ``computed`` tokens hit vLLM's own prefix cache."""
    req = SimpleNamespace(request_id=rid, prompt_token_ids=prompt)
    n, _ = conn.get_num_new_matched_tokens(req, computed)
    ids = list(block_ids) if block_ids is not None else [1000 + i for i in range(n_blocks)]
    blocks = SimpleNamespace(blocks=[[SimpleNamespace(block_id=i) for i in ids[:n_blocks]]])
    conn.update_state_after_alloc(req, blocks, n)
    meta = conn.build_connector_meta(SimpleNamespace(num_scheduled_tokens={rid: len(prompt)}))
    return n, meta.reqs_to_load.get(rid)


def test_scheduler_assembles_chunks_at_their_prompt_positions():
    rng = np.random.default_rng(2)
    a = rng.integers(0, 30000, size=528).tolist()  # 33 pages
    b = rng.integers(0, 30000, size=256).tolist()
    idx = ChunkAssemblyIndex(BS)
    run(idx.insert(meta_for(a, 40, pos_offset=0)))
    run(idx.insert(meta_for(b, 7, pos_offset=3000)))
    prompt = a + b + [5] * 20
    n, spec = _schedule(_scheduler(ServerWithIndex(idx)), "r", prompt, 60)
    assert n == 784
    assert spec.block_ids == list(range(1000, 1049))
    assert [(s.start_slot, s.num_slots, s.block_offset, s.pos_offset, s.new_pos)
            for s in spec.segments] == [(40, 33, 0, 0, 0), (7, 16, 33, 3000, 528)]
    plan = C.plan_load({"r": spec}, SLOT)
    # a: stored at 0, placed at 0 (copied); b: stored at 3000, placed at 528
    assert plan.deltas == [528 - 3000]
    assert plan.rope_idx.tolist() == [-1] * 33 + [0] * 16
    assert plan.page_ids.tolist() == list(range(1000, 1049))
    assert plan.reads == [(0, 33 * SLOT, 40 * SLOT), (33 * SLOT, 16 * SLOT, 7 * SLOT)]


def test_scheduler_prefix_index_hit_at_zero():
    """With the reference's single-prefix lookup, the hit is placed at 0."""
    rng = np.random.default_rng(3)
    a = rng.integers(0, 30000, size=160).tolist()
    idx = IncrementalPrefixIndex(BS)
    run(idx.insert(meta_for(a, 12, pos_offset=3000)))
    n, spec = _schedule(_scheduler(ServerWithIndex(idx)), "r", a + [1, 2, 3], 11)
    assert n == 160 and spec.segments == []
    assert (spec.start_slot, spec.num_slots, spec.pos_offset, spec.new_pos) == (12, 10, 3000, 0)


def test_place_chunks_stops_at_alternatives_and_misalignment():
    rng = np.random.default_rng(4)
    a = rng.integers(0, 100, size=64).tolist()
    b = rng.integers(0, 100, size=32).tolist()
    ch = lambda t, s: {"chunk_key": chunk_key(t), "start_slot": s, "num_slots": len(t) // BS,
                       "token_count": len(t), "pos_offset": 0, "file_offset": s * SLOT}
    # consecutive pieces
    assert [p for p, _ in C.place_chunks(a + b, [ch(a, 0), ch(b, 9)], BS)] == [0, 64]
    # an alternative (another prefix of the prompt) is not a consecutive piece
    assert [p for p, _ in C.place_chunks(a + b, [ch(a, 0), ch(a[:32], 5)], BS)] == [0]
    # a piece that would start off a block boundary is not placed
    odd = a[:40]
    rest = (a + b)[40:72]
    assert [p for p, _ in C.place_chunks(a + b, [ch(odd, 0), ch(rest, 3)], BS)] == [0]
    # the first chunk is trusted like the reference's hit; later ones verified
    assert C.place_chunks(a, [], BS) == []


def test_load_spec_clips_to_the_blocks_given():
    placed = [(0, {"chunk_key": "x", "start_slot": 4, "num_slots": 3, "token_count": 48,
                   "pos_offset": 0, "file_offset": 4 * SLOT}),
              (48, {"chunk_key": "y", "start_slot": 20, "num_slots": 4, "token_count": 64,
                    "pos_offset": 100, "file_offset": 20 * SLOT})]
    spec = C.load_spec(placed, [9, 8, 7, 6, 5], BS)
    assert [(s.num_slots, s.block_offset, s.new_pos) for s in spec.segments] == \
        [(3, 0, 0), (2, 3, 48)]
    # the second chunk is cut to 2 of its 4 pages: 80 tokens are loaded
    assert spec.block_ids == [9, 8, 7, 6, 5] and spec.token_count == 80
    one = C.load_spec(placed, [9, 8], BS)
    assert one.segments == [] and one.num_slots == 2 and one.block_ids == [9, 8]
    assert C.load_spec(placed, [], BS) is None


def test_load_spec_skips_the_blocks_vllm_computed():
    """Blocks below first_block hold vLLM's own prefix-cache KV: nothing is
    loaded there, and a cut segment keeps its rotation delta."""
    placed = [(0, {"chunk_key": "x", "start_slot": 4, "num_slots": 3, "token_count": 48,
                   "pos_offset": 0, "file_offset": 4 * SLOT}),
              (48, {"chunk_key": "y", "start_slot": 20, "num_slots": 4, "token_count": 64,
                    "pos_offset": 100, "file_offset": 20 * SLOT})]
    ids = [9, 8, 7, 6, 5, 4, 3]
    spec = C.load_spec(placed, ids, BS, first_block=2)
    assert spec.block_ids == [7, 6, 5, 4, 3] and spec.token_count == 112
    assert [(s.start_slot, s.num_slots, s.block_offset, s.pos_offset, s.new_pos)
            for s in spec.segments] == [(6, 1, 0, 32, 32), (20, 4, 1, 100, 48)]
    # the whole first chunk computed, and one page of the second
    spec = C.load_spec(placed, ids, BS, first_block=4)
    assert spec.block_ids == [5, 4, 3] and spec.segments == []
    assert (spec.start_slot, spec.num_slots, spec.pos_offset, spec.new_pos) == (21, 3, 116, 64)
    plan = C.plan_load({"r": spec}, SLOT)
    assert plan.deltas == [48 - 100] and plan.page_ids.tolist() == [5, 4, 3]
    assert C.load_spec(placed, ids, BS, first_block=7) is None


def test_scheduler_with_vllm_prefix_hit_loads_only_the_rest():
    """num_computed_tokens > 0 (vLLM's local prefix cache): the load fills
    the blocks from there on, and none of the computed ones."""
    rng = np.random.default_rng(6)
    a = rng.integers(0, 30000, size=528).tolist()  # 33 pages
    b = rng.integers(0, 30000, size=256).tolist()  # 16 pages
    idx = ChunkAssemblyIndex(BS)
    run(idx.insert(meta_for(a, 40, pos_offset=0)))
    run(idx.insert(meta_for(b, 7, pos_offset=3000)))
    prompt = a + b + [5] * 20
    n, spec = _schedule(_scheduler(ServerWithIndex(idx)), "r", prompt, 60, computed=80)
    assert n == 784 - 80
    assert spec.block_ids == list(range(1005, 1049))
    assert [(s.start_slot, s.num_slots, s.block_offset, s.pos_offset, s.new_pos)
            for s in spec.segments] == [(45, 28, 0, 80, 80), (7, 16, 28, 3000, 528)]
    plan = C.plan_load({"r": spec}, SLOT)
    assert plan.page_ids.tolist() == list(range(1005, 1049))
    assert plan.rope_idx.tolist() == [-1] * 28 + [0] * 16
    # vLLM computed past the first chunk: only the rest of the second loads
    n, spec = _schedule(_scheduler(ServerWithIndex(idx)), "s", prompt, 60, computed=560)
    assert n == 784 - 560 and spec.block_ids == list(range(1035, 1049))
    assert (spec.start_slot, spec.num_slots, spec.pos_offset, spec.new_pos) == \
        (9, 14, 3032, 560)
    # vLLM computed everything a hit would give: nothing to load
    n, spec = _schedule(_scheduler(ServerWithIndex(idx)), "t", prompt, 60, computed=784)
    assert n == 0 and spec is None


def test_chunk_assembly_is_opt_in():
    """Without allow_chunk_assembly only the first chunk of a reply loads,
    as the reference's single prefix hit."""
    rng = np.random.default_rng(7)
    a = rng.integers(0, 30000, size=64).tolist()
    b = rng.integers(0, 30000, size=64).tolist()
    idx = ChunkAssemblyIndex(BS)
    run(idx.insert(meta_for(a, 1, pos_offset=0)))
    run(idx.insert(meta_for(b, 9, pos_offset=0)))
    n, spec = _schedule(_scheduler(ServerWithIndex(idx), assemble=False), "r", a + b + [1], 9)
    assert n == 64 and spec.segments == [] and spec.block_ids == list(range(1000, 1004))
    n, spec = _schedule(_scheduler(ServerWithIndex(idx)), "r", a + b + [1], 9)
    assert n == 128 and len(spec.segments) == 2


def test_whole_prompt_hit_leaves_one_token_to_compute():
    """A cached chunk covering the whole (block-aligned) prompt reports one
    token less, so vLLM computes the last one; the load still covers every
    page of the chunk."""
    rng = np.random.default_rng(5)
    a = rng.integers(0, 30000, size=64).tolist()
    idx = IncrementalPrefixIndex(BS)
    run(idx.insert(meta_for(a, 3)))
    n, spec = _schedule(_scheduler(ServerWithIndex(idx)), "r", a, 8)
    assert n == 63
    assert spec.num_slots == 4 and spec.block_ids == [1000, 1001, 1002, 1003]
    assert (spec.pos_offset, spec.new_pos) == (0, 0)


# The reference's own index behaviours (tests/retrieval/test_prefix_index.py:
# exact hit, a longer query finds the prefix, miss, remove, model isolation),
# held by both indexes at block size 4.
@pytest.mark.parametrize("cls", [IncrementalPrefixIndex, ChunkAssemblyIndex])
def test_reference_index_behaviours(cls):
    toks = [1, 2, 3, 4]
    meta = ChunkMeta(chunk_key(toks), 0, 1, 4, 0, "m")
    idx = cls(4)
    assert run(idx.lookup(toks, "m")) == []
    run(idx.insert(meta))
    assert [m.chunk_key for m in run(idx.lookup(toks, "m"))] == [meta.chunk_key]
    assert [m.chunk_key for m in run(idx.lookup([1, 2, 3, 4, 5, 6, 7, 8], "m"))] == \
        [meta.chunk_key]
    assert run(idx.lookup(toks, "other-model")) == []
    run(idx.remove(meta.chunk_key))
    assert run(idx.lookup(toks, "m")) == []
