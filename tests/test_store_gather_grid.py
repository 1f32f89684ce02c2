"""The fused store+gather launch's grid split, on the host.

nkv_store_gather (csrc/nkv_store_gather.hip, sg_is_cached) interleaves its
new-row and cached-row workgroups: position b of a grid of G = N + C
workgroups is a cached-row workgroup when umulhi(b + 1, spread) >
umulhi(b, spread), spread = ceil(C * 2^32 / G), and its index within its
kind is umulhi(b, spread) (cached) or b - umulhi(b, spread) (new rows).
Every workgroup trusts that index to stay below its kind's count, so the
split must be a bijection onto [0, N) + [0, C) for every N >= 1, C >= 0
that a launch can have (G < 2^31).  Checked here with 64-bit integer
arithmetic, exhaustively on small grids and on the decode, chunked-prefill
and narrow-row launch sizes, and at the ends of very large grids."""
from __future__ import annotations

import numpy as np
import pytest


def spread_of(new: int, cached: int) -> int:
    total = new + cached
    return ((cached << 32) + total - 1) // total


def split(new: int, cached: int):
    total = new + cached
    m = np.uint64(spread_of(new, cached))
    b = np.arange(total, dtype=np.uint64)
    before = (b * m) >> np.uint64(32)
    after = ((b + np.uint64(1)) * m) >> np.uint64(32)
    is_cached = after > before
    return before[is_cached], (b - before)[~is_cached], is_cached


def _check_bijection(new: int, cached: int) -> None:
    assert spread_of(new, cached) < 2**32
    cached_index, new_index, _ = split(new, cached)
    np.testing.assert_array_equal(cached_index, np.arange(cached))
    np.testing.assert_array_equal(new_index, np.arange(new))


def test_split_is_a_bijection_on_small_grids():
    for new in range(1, 40):
        for cached in range(0, 40):
            _check_bijection(new, cached)


@pytest.mark.parametrize("new,cached", [(128, 890_000), (4096, 1904), (4584, 3904), (1, 7), (7, 1)])
def test_split_is_a_bijection_on_launch_sizes(new, cached):
    _check_bijection(new, cached)


def test_split_spreads_the_new_rows_evenly():
    """Between two new-row workgroups lie floor or ceil of C / N cached ones."""
    new, cached = 128, 890_000
    _, _, is_cached = split(new, cached)
    gaps = np.diff(np.flatnonzero(~is_cached)) - 1
    assert gaps.min() >= cached // new - 1 and gaps.max() <= -(-cached // new) + 1


@pytest.mark.parametrize("new,cached", [(1, 2**31 - 3), (2**30, 2**30 - 2), (7, 2**31 - 20)])
def test_split_ends_of_large_grids(new, cached):
    total, m = new + cached, spread_of(new, cached)
    assert m < 2**32
    assert (total * m) >> 32 == cached          # exactly C cached positions in [0, G)
    assert ((total - 1) * m) >> 32 <= cached     # indexes stay below C
