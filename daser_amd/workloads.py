"""Seeded synthetic workloads of the five benchmark configurations.

Each workload describes requests over a pool of paged KV blocks: how many
tokens each request holds, which (randomly permuted) blocks hold them, and
where each page's slot record sits in one contiguous staging arena (pages of
all requests back to back, so request r's chunk buffer is a contiguous
sub-range, exactly the per-request staging of the reference,
daser/connector/daser_connector.py:616-623). Everything here is host-side
numpy; device tensors are created by the callers.
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field
from typing import Optional

import numpy as np


@dataclass(frozen=True)
class KVShape:
    num_layers: int
    num_heads: int
    head_dim: int
    block_size: int
    elem_bytes: int  # 2 = bf16/fp16, 1 = e4m3

    @property
    def page_bytes(self) -> int:
        return self.block_size * self.num_heads * self.head_dim * self.elem_bytes

    @property
    def layer_bytes(self) -> int:
        return 2 * self.page_bytes

    @property
    def slot_bytes(self) -> int:
        return self.layer_bytes * self.num_layers


QWEN2_05B = KVShape(24, 2, 64, 16, 2)
LLAMA3_8B = KVShape(32, 8, 128, 16, 2)
LLAMA3_8B_FP8 = KVShape(32, 8, 128, 16, 1)
LLAMA3_70B = KVShape(80, 8, 128, 16, 2)
LLAMA3_70B_TP8 = KVShape(80, 1, 128, 16, 2)  # one rank's heads under 8-way tensor parallelism


@dataclass
class PagedWorkload:
    """Requests mapped onto a permuted block pool.

    page_ids[p]      block id of global page p (requests back to back)
    slot_offsets[p]  byte offset of page p's slot record in the staging arena
    req_pages[r]     pages of request r
    """

    shape: KVShape
    num_blocks: int
    req_tokens: list[int]
    req_pages: list[int]
    page_ids: np.ndarray
    slot_offsets: np.ndarray
    # re-rotation (RAG reuse): per-page source record offsets and deltas
    src_offsets: Optional[np.ndarray] = None
    page_delta: Optional[np.ndarray] = None
    chunk_pages: Optional[list[int]] = None
    chunk_delta: Optional[list[int]] = None
    meta: dict = field(default_factory=dict)

    @property
    def n_pages(self) -> int:
        return int(self.page_ids.size)

    @property
    def staging_bytes(self) -> int:
        return self.n_pages * self.shape.slot_bytes

    @property
    def payload_bytes(self) -> int:
        """P: K+V bytes of every page over every layer (one direction)."""
        return self.n_pages * self.shape.slot_bytes

    @property
    def tokens(self) -> int:
        return int(sum(self.req_tokens))


def ragged(shape: KVShape, n_req: int, lo: int, hi: int, seed: int,
           pool_slack: float = 1.0, num_blocks: Optional[int] = None) -> PagedWorkload:
    """Requests with lengths ~ U[lo, hi] tokens on a randomly permuted pool.

    Pages per request = ceil(tokens / block_size) (the reference moves whole
    pages, daser/connector/daser_connector.py:280). The pool holds
    ceil(total_pages * pool_slack) blocks unless num_blocks is given.
    """
    rng = np.random.default_rng(seed)
    toks = rng.integers(lo, hi + 1, size=n_req).tolist()
    pages = [math.ceil(t / shape.block_size) for t in toks]
    total = sum(pages)
    nb = num_blocks if num_blocks is not None else int(math.ceil(total * pool_slack))
    if nb < total:
        raise ValueError("block pool smaller than the requests' pages")
    perm = rng.permutation(nb)[:total].astype(np.int32)
    offs = np.arange(total, dtype=np.int64) * shape.slot_bytes
    return PagedWorkload(shape, nb, toks, pages, perm, offs)


def rag_reuse(shape: KVShape, n_req: int, chunks_per_req: int, chunk_tokens: int,
              n_src_chunks: Optional[int], max_offset: int, seed: int,
              pool_slack: float = 1.0) -> PagedWorkload:
    """Requests assembled from cached chunks re-inserted at new positions.

    Every cached chunk was stored at position 0 and occupies
    chunk_tokens / block_size slot records in the source arena. Request r's
    chunk c is source chunk ``src[r, c]`` (distinct chunks when n_src_chunks
    is None, else drawn from n_src_chunks shared ones) placed at a random new
    position in [0, max_offset); the delta to re-rotate by is that position.
    """
    rng = np.random.default_rng(seed)
    if chunk_tokens % shape.block_size:
        raise ValueError("chunk length must be a whole number of pages")
    cp = chunk_tokens // shape.block_size
    n_chunks = n_req * chunks_per_req
    if n_src_chunks is None:
        src = np.arange(n_chunks)
        n_src = n_chunks
    else:
        src = np.concatenate([rng.permutation(n_src_chunks)[: chunks_per_req]
                              if chunks_per_req <= n_src_chunks
                              else rng.integers(0, n_src_chunks, chunks_per_req)
                              for _ in range(n_req)])
        n_src = n_src_chunks
    deltas = rng.integers(0, max_offset, size=n_chunks).astype(np.int64)
    total = n_chunks * cp
    nb = int(math.ceil(total * pool_slack))
    perm = rng.permutation(nb)[:total].astype(np.int32)
    page_in_chunk = np.tile(np.arange(cp, dtype=np.int64), n_chunks)
    src_offsets = (np.repeat(src, cp) * cp + page_in_chunk) * shape.slot_bytes
    wl = PagedWorkload(
        shape, nb, [chunks_per_req * chunk_tokens] * n_req,
        [chunks_per_req * cp] * n_req, perm,
        np.arange(total, dtype=np.int64) * shape.slot_bytes,
        src_offsets=src_offsets.astype(np.int64),
        page_delta=np.repeat(deltas, cp),
        chunk_pages=[cp] * n_chunks,
        chunk_delta=deltas.tolist(),
    )
    wl.meta["n_src_chunks"] = n_src
    wl.meta["src_staging_bytes"] = n_src * cp * shape.slot_bytes
    return wl


# The five configurations of the benchmark plan.
def config(n: int, seed: int = 0) -> PagedWorkload:
    if n == 1:  # CPU plumbing: Qwen2-0.5B shape, pool of 1024 blocks
        return ragged(QWEN2_05B, 8, 100, 2000, seed, num_blocks=1024)
    if n == 2:  # Llama-3-8B gather -> scatter
        return ragged(LLAMA3_8B, 64, 512, 8192, seed, pool_slack=1.05)
    if n == 3:  # RAG chunk reuse with re-rotation
        return rag_reuse(LLAMA3_8B, 32, 10, 512, None, 32768, seed, pool_slack=1.05)
    if n == 4:  # fp8 e4m3 KV
        return ragged(LLAMA3_8B_FP8, 128, 256, 16384, seed, pool_slack=1.05)
    if n == 5:  # Llama-3-70B single-GPU share
        return rag_reuse(LLAMA3_70B, 16, 64, 512, 64, 32768, seed)
    if n == 6:  # the same workload as config 5, one TP8 rank's share (H = 1, 4 KiB pages)
        return rag_reuse(LLAMA3_70B_TP8, 16, 64, 512, 64, 32768, seed)
    raise ValueError(f"unknown config {n}")


CONFIG_NAMES = {
    1: "qwen2-0.5b paged gather+scatter round trip (L24 H2 D64 bs16 bf16, 8 req U[100,2000])",
    2: "llama-3-8b paged gather->scatter (L32 H8 D128 bs16 bf16, 64 req U[512,8192], 256-token chunk staging)",
    3: "llama-3-8b RAG reuse re-rotate+scatter (32 req x 10 x 512-token chunks, offset U[0,32768), theta 5e5)",
    4: "llama-3-8b fp8 e4m3 paged gather->scatter (128 req U[256,16384], per-layer scales)",
    5: "llama-3-70b single-GPU share re-rotate+scatter (L80, 16 x 32768 tokens from 64 reused 512-token chunks)",
    6: "llama-3-70b TP8 rank share re-rotate+scatter (L80 H1 D128, 4 KiB pages, config 5's requests)",
}
