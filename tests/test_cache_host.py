"""Host logic of the slot-indexed cache (gdn_replayssm_cache.ReplaySSMCache):
the step metadata it derives from the ring fills, as the reference's host
cycle sequences it (prototype/bench_gdn_full_contract.py:225-308): ring slot
pos = fill, valid_len = fill + 1, flush when the ring is full, ring restarted
after it; padding entries (slot 0) append nothing, replay nothing, never
flush. No GPU: only the metadata is exercised."""

from __future__ import annotations

import numpy as np
import pytest

from gdn_replayssm_cache import ReplaySSMCache


def _cache(num_slots=5, window=4):
    return ReplaySSMCache(num_slots, window, heads=2, value_heads=4, key_dim=128, value_dim=32, device="cpu")


def _advance(cache, slots):
    """What step() does to the fills, without a launch."""
    slots, pos, valid, flush = cache.metadata(slots)
    live = slots != 0
    cache.fill[slots[live]] = np.where(flush, 0, valid)[live]
    return pos, valid, flush


def test_fill_cycle_and_flush():
    cache = _cache()
    seen = []
    for _ in range(9):
        pos, valid, flush = _advance(cache, [3])
        seen.append((int(pos[0]), int(valid[0]), bool(flush[0])))
    assert seen == [(0, 1, False), (1, 2, False), (2, 3, False), (3, 4, True),
                    (0, 1, False), (1, 2, False), (2, 3, False), (3, 4, True), (0, 1, False)]


def test_padding_and_phases():
    cache = _cache()
    _advance(cache, [1])
    _advance(cache, [1, 2])
    pos, valid, flush = _advance(cache, [2, 0, 1, 0])
    assert pos.tolist() == [1, -1, 2, -1]
    assert valid.tolist() == [2, 0, 3, 0]
    assert flush.tolist() == [False, False, False, False]
    assert cache.fill[0] == 0


def test_release_restarts_the_ring():
    cache = _cache()
    for _ in range(3):
        _advance(cache, [4])
    cache.release(4)
    pos, valid, _ = _advance(cache, [4])
    assert (pos[0], valid[0]) == (0, 1)


@pytest.mark.parametrize("slots", [[1, 1], [0, 6], [-1]])
def test_bad_batches_are_rejected(slots):
    with pytest.raises(ValueError):
        _cache().metadata(slots)


def test_padding_may_repeat():
    _cache().metadata([0, 0, 2])
