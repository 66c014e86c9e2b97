"""Position encoders (reference daser/position/) and how a stored offset
turns into the re-rotation delta of a load."""

from types import SimpleNamespace

import numpy as np
import pytest

from daser_amd import connector as C
from daser_amd.position import FixedOffsetEncoder, PrefillOffsetEncoder


def test_fixed_offset_encoder_reference_semantics():
    # daser/position/fixed_offset.py:23-50: same offset for every chunk;
    # get_offset returns what ChunkMeta stored
    enc = FixedOffsetEncoder(7)
    assert enc.assign_offset("a", 16) == 7 and enc.assign_offset("b", 512) == 7
    assert enc.get_offset(SimpleNamespace(pos_offset=123)) == 123
    assert FixedOffsetEncoder().assign_offset("c", 1) == 0


def test_prefill_offset_encoder_records_positions_once():
    enc = PrefillOffsetEncoder()
    enc.note_position("passage", 3000)
    assert enc.assign_offset("prefix", 256) == 0      # never noted: default
    assert enc.assign_offset("passage", 512) == 3000
    assert enc.assign_offset("passage", 512) == 0     # consumed
    assert enc.get_offset(SimpleNamespace(pos_offset=3000)) == 3000
    with pytest.raises(ValueError):
        enc.note_position("x", -1)


def test_stored_offset_becomes_load_delta():
    """A passage prefilled at 3000 and reused at 500 is rotated by -2500;
    one reused at its own position is a plain copy."""
    enc = PrefillOffsetEncoder()
    enc.note_position("p", 3000)
    stored = enc.assign_offset("p", 512)
    meta = SimpleNamespace(pos_offset=stored)
    slot = 1 << 16
    reqs = {
        "moved": C.ReqLoadSpec("p", 4, 32, list(range(32)), 4 * slot, 512,
                               pos_offset=enc.get_offset(meta), new_pos=500),
        "same": C.ReqLoadSpec("p", 4, 32, list(range(32, 64)), 4 * slot, 512,
                              pos_offset=enc.get_offset(meta), new_pos=3000),
    }
    plan = C.plan_load(reqs, slot)
    assert plan.deltas == [-2500]
    assert np.array_equal(plan.rope_idx, np.r_[np.zeros(32, np.int32), -np.ones(32, np.int32)])
