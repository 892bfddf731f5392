"""Pins oracle.permute by a brute-force double loop."""
import numpy as np

from oracle.permute import permute


def _brute(ids, E):
    T, k = ids.shape
    order = []
    for e in range(E):
        for t in range(T):
            for j in range(k):
                if ids[t, j] == e:
                    order.append(t * k + j)
    return np.array(order, np.int32)


def test_permute_matches_brute_force():
    rng = np.random.default_rng(0)
    for T, k, E in [(1, 1, 4), (7, 3, 16), (50, 4, 9), (0, 2, 3)]:
        ids = np.stack([rng.permutation(E)[:k] for _ in range(T)]) if T else \
            np.zeros((0, k), np.int64)
        p = permute(ids, E)
        order = _brute(ids, E)
        np.testing.assert_array_equal(p["sorted_idx"], order)
        np.testing.assert_array_equal(p["counts"], np.bincount(ids.ravel(), minlength=E))
        assert p["offsets"][0] == 0 and p["offsets"][-1] == T * k
        np.testing.assert_array_equal(p["sorted_idx"][p["inv_pos"]], np.arange(T * k))
