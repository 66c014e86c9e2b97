"""One-pass prefix keys equal the reference's per-prefix hashes."""

import numpy as np

from daser_amd.connector import hash_tokens
from daser_amd.prefix_hash import prefix_keys


def test_keys_equal_per_prefix_hashes():
    rng = np.random.default_rng(0)
    toks = rng.integers(0, 150_000, size=1000).tolist()
    keys = prefix_keys(toks, 16)
    assert len(keys) == 1000 // 16
    for i, k in enumerate(keys):
        assert k == hash_tokens(toks[: (i + 1) * 16])


def test_short_and_negative_tokens():
    assert prefix_keys([1, 2, 3], 16) == []
    toks = [-1, 2 ** 31 - 1, 0, 7] * 4
    assert prefix_keys(toks, 4)[-1] == hash_tokens(toks)


def test_numpy_input_equals_list_input():
    toks = np.arange(-50, 270, dtype=np.int64)
    assert prefix_keys(toks, 16) == prefix_keys(toks.tolist(), 16)
