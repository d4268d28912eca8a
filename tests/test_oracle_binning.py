"""Pins the oracle's binning (duplication + stable sort + tile ranges) against
brute force: every (tile, gaussian) pair enumerated in the reference's
duplication order (gaussian-major, tiles z->y->x; bin_and_sort_gaussians.cu:11-35),
sorted with Python's sorted() on (tile, gaussian) — what a stable sort of the
gaussian-major sequence by tile gives — and run-length tile ranges."""
import numpy as np
import pytest

import oracle as O


def _random_boxes(rng, n, Tx, Ty, Tz, empty_frac=0.2):
    lo = np.stack([rng.integers(0, T, n) for T in (Tx, Ty, Tz)], 1)
    ext = np.stack([rng.integers(1, 4, n) for _ in range(3)], 1)
    hi = np.minimum(lo + ext, [Tx, Ty, Tz])
    empty = rng.random(n) < empty_frac
    lo[empty] = 0
    hi[empty] = 0
    return lo.astype(np.int32), hi.astype(np.int32)


def _brute(lo, hi, Tx, Ty, Tz):
    pairs = []
    for g in range(lo.shape[0]):
        for z in range(lo[g, 2], hi[g, 2]):
            for y in range(lo[g, 1], hi[g, 1]):
                for x in range(lo[g, 0], hi[g, 0]):
                    pairs.append((z * Ty * Tx + y * Tx + x, g))
    order = sorted(pairs)
    ids = np.array([g for _, g in order], np.int32)
    bins = np.zeros((Tx * Ty * Tz, 2), np.int32)
    for i, (t, _) in enumerate(order):
        if i == 0 or order[i - 1][0] != t:
            bins[t, 0] = i
        bins[t, 1] = i + 1
    return ids, bins, np.array([t for t, _ in order], np.int32)


@pytest.mark.parametrize("vol,n,seed", [((20, 24, 17), 60, 0), ((64, 8, 8), 40, 1),
                                        ((5, 5, 5), 30, 2), ((40, 40, 40), 300, 3)])
def test_bin_and_sort_equals_brute_force(vol, n, seed):
    rng = np.random.default_rng(seed)
    Tx, Ty, Tz = O.tile_grid(vol)
    lo, hi = _random_boxes(rng, n, Tx, Ty, Tz)
    cnt = np.prod(np.maximum(hi - lo, 0), axis=1).astype(np.int32)
    cum = O.cumsum(cnt)
    np.testing.assert_array_equal(cum, np.cumsum(cnt))
    ids, bins, keys = O.bin_and_sort(n, int(cum[-1]), lo, hi, cum, vol, return_keys=True)
    rids, rbins, rkeys = _brute(lo, hi, Tx, Ty, Tz)
    np.testing.assert_array_equal(ids, rids)
    np.testing.assert_array_equal(bins, rbins)
    np.testing.assert_array_equal(keys, rkeys)


def test_bin_and_sort_empty_and_inconsistent():
    z = np.zeros((4, 3), np.int32)
    ids, bins = O.bin_and_sort(4, 0, z, z, np.zeros(4, np.int32), (16, 16, 16))
    assert ids.size == 0 and not bins.any()
    lo = np.zeros((1, 3), np.int32)
    hi = np.ones((1, 3), np.int32)
    with pytest.raises(RuntimeError):  # cum[-1] must equal num_intersects
        O.bin_and_sort(1, 5, lo, hi, np.array([1], np.int32), (16, 16, 16))
