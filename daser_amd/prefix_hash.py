"""Block-aligned prefix keys in one pass.

The reference keys a cached chunk by ``xxh3_128(bytes(array('i', tokens)))``
(daser/connector/daser_connector.py:41-57, daser/retrieval/prefix.py:17-30)
and finds the longest cached prefix by hashing every block-aligned prefix
from scratch, longest first (daser/retrieval/prefix.py:49-72): O(n^2 / bs)
bytes hashed per lookup, a cold-path cost its own notes list as open. The
xxh3 streaming state gives the digest of each prefix as the tokens are fed
once, so all n / bs keys cost one pass, and they are the same keys.
daser_amd.retrieval builds its lookups on them.
"""

from __future__ import annotations

from typing import Iterable

import numpy as np


def prefix_keys(tokens: Iterable[int], block_tokens: int) -> list[str]:
    """Keys of the prefixes of length bs, 2 bs, ..., floor(n / bs) * bs, equal
    to ``hash_tokens(tokens[:k])`` of the reference for each k."""
    import xxhash

    if block_tokens <= 0:
        raise ValueError("block_tokens must be positive")
    arr = tokens if isinstance(tokens, np.ndarray) else np.asarray(list(tokens))
    buf = np.ascontiguousarray(arr, dtype=np.int32).tobytes()
    step = 4 * block_tokens
    h = xxhash.xxh3_128()
    keys = []
    for off in range(0, len(buf) - step + 1, step):
        h.update(buf[off:off + step])
        keys.append(h.hexdigest())
    return keys
