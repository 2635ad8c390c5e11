"""Selection indices are bit-exact with the oracle (src/kvssd/selectors.py:11-28)."""

import random

import pytest

from kvssd.selectors import AllBlocks, RecentSinkBlocks
from oracle import oracle as O


def test_known_answers():
    assert RecentSinkBlocks(1, 32).select(list(range(2048))) == [0] + list(range(2016, 2048))
    assert RecentSinkBlocks(1, 0).select([0, 1, 2]) == [0]
    assert RecentSinkBlocks(2, 2).select([0, 1, 2]) == [0, 1, 2]
    with pytest.raises(ValueError):
        RecentSinkBlocks(-1, 2).select([0])


def test_random_lists_match_oracle():
    rng = random.Random(0)
    for _ in range(500):
        n = rng.randint(0, 40)
        avail = sorted(rng.sample(range(200), n))
        sink, recent = rng.randint(0, 45), rng.randint(0, 45)
        assert RecentSinkBlocks(sink, recent).select(avail) == O.select_recent_sink(avail, sink, recent)
        assert AllBlocks().select(avail) == O.select_all(avail)
