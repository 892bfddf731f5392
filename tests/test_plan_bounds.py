"""CPU checks of the streamed GEMMs' work-item sizing (no GPU needed).

The persistent launches hold at most 32 work items per workgroup; the host
sizes the grid from a bound of the ragged tile count. These tests take
C5-sized routings (T=16384, top-10, E=512, 128-row tiles) including the
adversarial ones, count tiles by brute force, and deal the items over the
grid the library picks exactly as the kernels do (XCD x = workgroup % 8
owns items [total x / 8, total (x + 1) / 8), dealt round-robin over its
workgroups), asserting no workgroup gets more than 32.
"""
import numpy as np
import pytest

from sllm_amd import _lib

ST_MAX_ITEMS = 32


def _need_lib():
    if not _lib.available():
        pytest.fail(f"library not built: {_lib._lib_error}")
    return _lib.lib()


def _max_items_per_workgroup(total: int, grid: int) -> int:
    nx = grid // 8
    worst = 0
    for x in range(8):
        beg, end = total * x // 8, total * (x + 1) // 8
        n = end - beg
        # workgroup j of this XCD takes items beg + j, beg + j + nx, ...
        worst = max(worst, -(-n // nx) if n else 0)
    return worst


def _counts_cases(N, E, k, rng):
    T = N // k
    yield "uniform", np.bincount(rng.integers(0, E, N), minlength=E)
    hot = np.zeros(E, np.int64)
    hot[:k] = T  # every token on the same k experts
    yield "all-on-k", hot
    z = 1.0 / np.arange(1, E + 1) ** 1.2
    yield "zipf", np.bincount(rng.choice(E, N, p=z / z.sum()), minlength=E)
    # the bound's extreme: as many experts as possible with one row, the
    # rest on one expert (sum ceil = touched + floor((N - touched) / bm))
    ext = np.ones(E, np.int64)
    ext[0] = N - (E - 1)
    yield "ones+one", ext
    # every touched expert just past a tile boundary
    over = np.full(E, 129, np.int64)
    over[0] += N - over.sum()
    yield "129-each", over


@pytest.mark.parametrize("bm", [128, 16, 32])
def test_tile_bound_covers_worst_routings(bm):
    lib = _need_lib()
    rng = np.random.default_rng(0)
    T, k, E = 16384, 10, 512
    N = T * k
    bound = lib.sllm_moe_tile_bound(N, E, bm)
    assert bound > 0
    for name, counts in _counts_cases(N, E, k, rng):
        assert counts.sum() == N and (counts >= 0).all(), name
        tiles = int(np.sum(-(-counts // bm)))
        assert tiles <= bound, (name, tiles, bound)
    # the bound is reached by the ones+one routing: it cannot be smaller
    ext = np.ones(E, np.int64)
    ext[0] = N - (E - 1)
    assert int(np.sum(-(-ext // bm))) == bound


@pytest.mark.parametrize("ncu", [256, 304, 80, 8])
def test_stream_grid_deals_at_most_32_items(ncu):
    lib = _need_lib()
    rng = np.random.default_rng(1)
    T, k, E, H, I = 16384, 10, 512, 2048, 512
    N = T * k
    bound = lib.sllm_moe_tile_bound(N, E, 128)
    sh_tiles = -(-T // 128)
    for slabs in (I // 128, H // 256):  # gate/up, then down
        upper = bound * slabs + sh_tiles * slabs
        grid = lib.sllm_moe_stream_grid(upper, ncu)
        assert grid % 8 == 0 and grid >= ncu
        for name, counts in _counts_cases(N, E, k, rng):
            total = (int(np.sum(-(-counts // 128))) + sh_tiles) * slabs
            assert _max_items_per_workgroup(total, grid) <= ST_MAX_ITEMS, (name, total)
        # the bound itself, and a decode-style split of it
        assert _max_items_per_workgroup(upper, grid) <= ST_MAX_ITEMS
        g3 = lib.sllm_moe_stream_grid(upper * 3, ncu)
        assert _max_items_per_workgroup(upper * 3, g3) <= ST_MAX_ITEMS
