"""Work-item coverage of the grouped GEMM launches (mr_grouped.hip, mr_grouped_q4k.hip).

Workgroup b takes work item (b mod 8) * ceil(n_work / 8) + b / 8, so that each XCD (b mod 8)
runs one contiguous range of items and their shared weights meet in its L2. Every item must be
taken by exactly one workgroup; the launch grid is the item bound rounded up to a multiple of 8
(grouped_grid). A grid of exactly the item bound leaves items out whenever n_work is not a
multiple of 8 and the grid is not at least 8 * ceil(n_work / 8) (the case below).
"""
import numpy as np
import pytest


def taken(grid: int, n_work: int) -> np.ndarray:
    per_xcd = (n_work + 7) // 8
    b = np.arange(grid)
    loc, w = b // 8, (b % 8) * per_xcd + b // 8
    ok = (loc < per_xcd) & (w < n_work)
    return np.bincount(w[ok], minlength=n_work)


def grouped_grid(items: int) -> int:
    return (items + 7) // 8 * 8


@pytest.mark.parametrize("seed", range(20))
def test_every_item_taken_once(seed):
    rng = np.random.default_rng(seed)
    for _ in range(200):
        n_rt = int(rng.integers(1, 40))
        max_tiles = int(rng.integers(1, 200))
        n_work = n_rt * int(rng.integers(1, max_tiles + 1))  # n_rt * tile_off[E] <= n_rt * max_tiles
        counts = taken(grouped_grid(n_rt * max_tiles), n_work)
        assert (counts == 1).all(), (n_rt, max_tiles, n_work)


def test_unrounded_grid_misses_items():
    # n_work = 9 items on a grid of 10: XCD ranges of 2 items, items 5 and 7 have no workgroup
    counts = taken(10, 9)
    assert list(np.nonzero(counts == 0)[0]) == [5, 7]
    assert (taken(grouped_grid(10), 9) == 1).all()
