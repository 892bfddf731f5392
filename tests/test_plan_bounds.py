"""CPU checks of the streamed GEMMs' work-item sizing (no GPU needed).

The decode kernel (moe_stream_dec_kernel) holds at most 32 work items per
workgroup; the prefill kernel (moe_stream_kernel) takes its items 32 at a
time and so has no limit, but must still take every item exactly once. The
host sizes each persistent grid from a bound of the ragged tile count. These
tests port the kernels' dealing exactly:

* prefill, weights through L2 (ranges): XCD x = workgroup % 8 owns items
  [total x / 8, total (x + 1) / 8), dealt round-robin over its workgroups;
* prefill, streamed weights, and every decode launch: items go to the XCDs
  in chunks of CB consecutive items (chunk c to XCD c % 8, the partial last
  chunk to XCD (total / CB) % 8), then round-robin over each XCD's
  workgroups; CB is one row tile's items of the first segment (column slabs,
  times K chunks in decode), an eighth of that (rounded up) in decode
  launches whose first segment has identity rows (the DeepSeek shared
  expert, a one-expert layer), and in decode at most a 64th of the
  launch's item bound.

They take the library's own plans (sllm_moe_plan_query: tile rows, K
splits, item bounds, deal chunks and grids) for decode batches of the
bench's shapes and of others, and assert that every tile count up to the
plan's bound deals no workgroup more than 32 items.
"""
import ctypes

import numpy as np
import pytest

from sllm_amd import _lib

ST_MAX_ITEMS = 32
PLAN_FIELDS = 22


def _need_lib():
    if not _lib.available():
        pytest.fail(f"library not built: {_lib._lib_error}")
    return _lib.lib()


def _xcd_count(total, xcd, cb, ranges):
    """Items XCD `xcd` owns (the kernels' xcount)."""
    if ranges:
        return total * (xcd + 1) // 8 - total * xcd // 8
    ncf, crem = divmod(total, cb)
    full = (ncf - xcd + 7) // 8 if ncf > xcd else 0
    return full * cb + (crem if ncf % 8 == xcd else 0)


def _item_at(total, xcd, q, cb, ranges):
    """Flat item index of the XCD's q-th item (the kernels' item_at)."""
    if ranges:
        return total * xcd // 8 + q
    return (xcd + 8 * (q // cb)) * cb + q % cb


def _deal(total, grid, cb, ranges):
    """Items of every workgroup, as lists of flat item indices."""
    nx = grid // 8
    out = []
    for b in range(grid):
        xcd, jx = b % 8, b // 8
        xc = _xcd_count(total, xcd, cb, ranges)
        n = (xc - jx + nx - 1) // nx if xc > jx else 0
        out.append([_item_at(total, xcd, jx + m * nx, cb, ranges) for m in range(n)])
    return out


def _max_items(total, grid, cb, ranges=False):
    """Most items one workgroup receives (workgroup jx = 0 of each XCD)."""
    nx = grid // 8
    return max(-(-_xcd_count(total, x, cb, ranges) // nx) for x in range(8))


@pytest.mark.parametrize("ranges", [False, True])
@pytest.mark.parametrize("cb", [1, 4, 8, 12, 96])
def test_deal_takes_every_item_once(ranges, cb):
    """The ported deal is a partition of [0, total) for every total."""
    for grid in (8, 64, 256):
        for total in list(range(0, 200)) + [1023, 4097]:
            items = sorted(i for w in _deal(total, grid, cb, ranges) for i in w)
            assert items == list(range(total)), (grid, total, cb, ranges)


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
def test_stream_dec_grid_deals_at_most_32_items(ncu):
    """The chunk-dealt grid bound holds for every total up to the bound,
    for chunk sizes of one tile's slabs (x K chunks)."""
    lib = _need_lib()
    for upper in (1, 31, 257, 4000, 9408, 20000):
        for cb in (1, 2, 4, 8, 12, 14, 28, 96, 160):
            grid = lib.sllm_moe_stream_dec_grid(upper, ncu, cb)
            assert grid % 8 == 0 and grid >= ncu
            worst = max(_max_items(t, grid, cb) for t in
                        range(max(0, upper - 3 * cb * 8), upper + 1))
            assert worst <= ST_MAX_ITEMS, (upper, cb, grid, worst)


def _sk_lreq(KB, w, ks):
    """Least stream-K range length keeping a unit within ks ranges."""
    return max(w, ((KB - 1) * w + ks - 2) // (ks - 1))


def _sample_tiles(max_tiles):
    """Routed tile counts to deal: the ends and a spread in between."""
    return sorted({1, 2, 3, max_tiles // 3, max_tiles // 2, max_tiles - 1,
                   max_tiles} - {0})


def _check_sk_deal(nu, KB, w, ks, grid, where):
    """Port of moe_stream_dec_kernel's stream-K deal: units of segment s
    (routed first) cost KB[s] w[s] on one line cut into G equal ranges, one
    per workgroup; a workgroup's items are the K steps of each unit whose
    start lies in its range. Checks that every unit's steps are dealt
    exactly once, in slices 0..P-1 with P <= ks (the first item zero-fills
    the rest), and that no workgroup meets more than 64 candidate units or
    holds more than 32 items."""
    assert grid % 8 == 0 and grid > 0, where
    c = [KB[s] * w[s] for s in range(len(nu))]
    cs = nu[0] * c[0]
    C = cs + (nu[1] * c[1] if len(nu) > 1 else 0)
    lreq = max(_sk_lreq(KB[s], w[s], ks[s]) for s in range(len(nu)))
    G = max(1, min(grid, C // lreq))

    def unit_of(x):
        return x // c[0] if x < cs else nu[0] + (x - cs) // c[1]

    def range_of(x):
        return ((x + 1) * G - 1) // C

    seen = {}
    for r in range(G):
        a, b = r * C // G, (r + 1) * C // G
        ua = unit_of(a)
        ncand = unit_of(b - 1) - ua + 1
        assert ncand <= 64, (where, r, ncand)
        items = 0
        for u in range(ua, ua + ncand):
            seg = int(u >= nu[0])
            li = u - nu[0] if seg else u
            cu = cs + li * c[1] if seg else li * c[0]
            kb, ww = KB[seg], w[seg]
            jlo = 0 if a <= cu else (a - cu + ww - 1) // ww
            jhi = min(kb, (b - cu + ww - 1) // ww)
            if jlo >= jhi:
                continue
            items += 1
            rfirst = range_of(cu)
            nsl = range_of(cu + (kb - 1) * ww) - rfirst + 1
            slot = r - rfirst
            fill = ks[seg] - nsl if slot == 0 else 0
            assert 0 <= slot < nsl <= ks[seg] and fill >= 0, (where, r, u)
            seen.setdefault(u, []).append((slot, jlo, jhi, fill))
        assert items <= ST_MAX_ITEMS, (where, r, items)
    assert len(seen) == sum(nu), where
    for u, pieces in seen.items():
        kb = KB[int(u >= nu[0])]
        pieces.sort()
        assert [p_[0] for p_ in pieces] == list(range(len(pieces))), (where, u)
        assert pieces[0][1] == 0 and pieces[-1][2] == kb, (where, u)
        for p0, p1 in zip(pieces, pieces[1:]):
            assert p0[2] == p1[1], (where, u)  # the steps tile the unit


def _chunk_cap(cb, upper):
    """A deal chunk holds at most a 64th of the launch's items (at least 1)."""
    return max(1, min(cb, upper // 64))


def _plan(lib, ds, T, H, E, I, Is, k, mode=2, logits_given=0):
    out = (ctypes.c_long * PLAN_FIELDS)()
    rc = lib.sllm_moe_plan_query(ds, T, H, E, I, Is, k, mode, logits_given,
                                 ctypes.addressof(out), PLAN_FIELDS)
    assert rc == 0, _lib.last_error()
    return list(out)


# (deepseek, H, E, k, I, Is): the bench's C3 shape, the DeepSeek C4 shape,
# and shapes whose decode plans split the down projection finely
SHAPES = [
    (0, 2048, 512, 10, 512, 512),      # C2 / C3
    (0, 4096, 128, 8, 1536, 1536),     # a Qwen3-style layer
    (0, 3584, 64, 8, 2560, 20480),     # a wide shared expert
    (0, 2048, 64, 6, 1408, 5632),
    (0, 5120, 1, 1, 17408, 0),         # a dense MLP run as the layer
    (1, 7168, 256, 8, 2048, 2048),     # C4
    (1, 4096, 64, 6, 1536, 1536),
]


@pytest.mark.parametrize("streamk", ["1", "0"])
@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: "x".join(map(str, s)))
def test_decode_plans_deal_at_most_32_items(shape, streamk, monkeypatch):
    """Every decode launch of the library's plans, at every batch size and
    every routed tile count up to the plan's bound (sampled for stream-K
    deals), deals no workgroup more than 32 items; with stream-K
    (SLLM_MOE_STREAMK=1, the default) every unit's K steps exactly once."""
    monkeypatch.setenv("SLLM_MOE_STREAMK", streamk)
    lib = _need_lib()
    ds, H, E, k, I, Is = shape
    for T in range(1, 65):
        p = _plan(lib, ds, T, H, E, I, Is, k)
        assert p[0] == 1
        bm, bm_sh, max_tiles = p[1], p[2], p[3]
        ks_up, ks_up_sh, ks_dn, ks_dn_sh = p[5], p[6], p[7], p[8]
        sh_rt = -(-T // bm_sh) if Is else 0
        # a DeepSeek shared expert with taller tiles than the routed ones
        # runs in launches of its own; otherwise it is the routed launches'
        # second segment
        sep = bool(ds and Is and bm_sh != bm)
        # per launch: (routed tiles -> items, shared items)
        launches = [
            (I // 128 * ks_up, (0 if sep else sh_rt * (Is // 128) * ks_up_sh)),
            (H // 256 * ks_dn, (0 if sep else sh_rt * (H // 256) * ks_dn_sh)),
        ]
        for j, (per_tile, shared) in enumerate(launches):
            upper, cb, grid = p[10 + 3 * j], p[11 + 3 * j], p[12 + 3 * j]
            assert upper == max_tiles * per_tile + shared, (T, j)
            if cb == 0:  # stream-K deal
                up = j == 0
                nu = [0, (sh_rt * (Is // 128 if up else H // 256)) if not sep else 0]
                KB = [H // 128 if up else I // 128, H // 128 if up else max(1, Is // 128)]
                w = [1, 2 if ds else 1]
                ks = [ks_up if up else ks_dn, ks_up_sh if up else ks_dn_sh]
                nseg = 2 if nu[1] else 1
                for rt in _sample_tiles(max_tiles):
                    nu[0] = rt * (I // 128 if up else H // 256)
                    _check_sk_deal(nu[:nseg], KB[:nseg], w[:nseg], ks[:nseg],
                                   grid, (T, j, rt))
                continue
            # identity rows (a one-expert layer): an eighth of a tile
            want_cb = per_tile if (ds or E > 1 or k > 1) else -(-per_tile // 8)
            assert cb == _chunk_cap(want_cb, upper) and grid % 8 == 0, (T, j)
            worst = max(_max_items(rt * per_tile + shared, grid, cb)
                        for rt in range(1, max_tiles + 1))
            assert worst <= ST_MAX_ITEMS, (T, j, upper, cb, grid, worst)
        if not sep:
            assert p[16] == p[19] == 0, T  # no launches of its own
        else:
            for j, per_tile in ((2, Is // 128 * ks_up_sh), (3, H // 256 * ks_dn_sh)):
                upper, cb, grid = p[10 + 3 * j], p[11 + 3 * j], p[12 + 3 * j]
                assert upper == sh_rt * per_tile
                if cb == 0:  # stream-K deal
                    units = sh_rt * (Is // 128 if j == 2 else H // 256)
                    KB = H // 128 if j == 2 else Is // 128
                    _check_sk_deal([units], [KB], [1], [ks_up_sh if j == 2 else ks_dn_sh],
                                   grid, (T, j))
                    continue
                assert cb == _chunk_cap(-(-per_tile // 8), upper), (T, j)
                assert _max_items(upper, grid, cb) <= ST_MAX_ITEMS, (T, j)


def test_old_contiguous_sizing_would_overflow(monkeypatch):
    """Regression: sizing the decode grid as if each XCD held a contiguous
    eighth of the items (sllm_moe_stream_grid) deals 37 items to a
    workgroup of the H 4096, E 128, top-8, I 1536 layer at 6 tokens, and
    36 to the H 3584, E 64, I 2560, Is 20480 layer at 7 tokens; the
    chunk-aware grid the library now launches keeps them at 32. (The old
    deal's chunks were whole row tiles; the library's are now capped at a
    64th of the items. The plans here deal whole items and take the
    count-based K splits, as they did then: SLLM_MOE_STREAMK=0,
    SLLM_MOE_SPLIT_DEALT=0.)"""
    monkeypatch.setenv("SLLM_MOE_STREAMK", "0")
    monkeypatch.setenv("SLLM_MOE_SPLIT_DEALT", "0")
    lib = _need_lib()
    for (ds, H, E, k, I, Is), T, old_worst in (
            ((0, 4096, 128, 8, 1536, 1536), 6, 37),
            ((0, 3584, 64, 8, 2560, 20480), 7, 36)):
        p = _plan(lib, ds, T, H, E, I, Is, k)
        bad = None
        for j in (0, 1):
            upper, cb, grid = p[10 + 3 * j], p[11 + 3 * j], p[12 + 3 * j]
            tile_cb = (I // 128 * p[5], H // 256 * p[7])[j]
            old = lib.sllm_moe_stream_grid(upper, p[9])
            w_old = _max_items(upper, old, tile_cb)
            if w_old > ST_MAX_ITEMS:
                bad = w_old
            if cb:  # (a stream-K launch, chunk 0, is checked by its port)
                assert _max_items(upper, grid, cb) <= ST_MAX_ITEMS
        assert bad == old_worst, (H, T, bad)


@pytest.mark.parametrize("ncu", [256, 304, 80, 8])
def test_prefill_grid_deals_every_item(ncu):
    """Prefill launches run one workgroup per CU (items taken 32 at a time):
    the ported deal covers every item once at C5-sized item counts."""
    lib = _need_lib()
    rng = np.random.default_rng(1)
    T, k, E, H, I = 16384, 10, 512, 2048, 512
    N = T * k
    sh_tiles = -(-T // 128)
    grid = 8 * (-(-ncu // 8))
    for slabs in (I // 128, H // 256):  # gate/up, then down
        for name, counts in _counts_cases(N, E, k, rng):
            total = (int(np.sum(-(-counts // 128))) + sh_tiles) * slabs
            for ranges in (False, True):
                dealt = _deal(total, grid, slabs, ranges)
                assert sum(len(w) for w in dealt) == total, name
                assert len({i for w in dealt for i in w}) == total, name


@pytest.mark.parametrize("H", [1024, 2048, 4096, 5120, 7168, 16384])
def test_decode_router_chunks_one_load_round_per_wave(H):
    """The decode router splits K into at least 2 chunks and enough that a
    workgroup's 8 waves take at most four 32-wide K slices each (one round
    of loads): 2 chunks at H = 2048 (C3), 7 at H = 7168 (C4); prefill-size
    batches (T > 64) keep one. Read from the DeepSeek plan, whose decode
    batches all route from the split logits."""
    lib = _need_lib()
    E, k, I = 256, 8, 2048
    for T in (1, 8, 16, 32, 64, 65):
        ks = _plan(lib, 1, T, H, E, I, I, k)[4]
        if T > 64:
            assert ks == 1, (H, T, ks)
            continue
        slices = H // 32
        assert ks >= 2 and -(-slices // ks) <= 32, (H, T, ks)
        # and no more than that: one chunk fewer would need a second round
        if ks > 2:
            assert -(-slices // (ks - 1)) > 32, (H, T, ks)
    assert _plan(lib, 1, 1, 2048, E, I, I, k)[4] == 2
    assert _plan(lib, 1, 1, 7168, E, I, I, k)[4] == 7


def _dealt_steps(exp_items, upper_items, tile_items, KB, ks, ncu=256):
    """The busiest workgroup's K steps under a decode launch's row-tile
    chunk deal (chunks of min(tile_items ks, upper ks / 64) items to the 8
    XCDs in turn, round-robin over an XCD's workgroups; the grid sized from
    the bound upper_items)."""
    n, nu = exp_items * ks, upper_items * ks
    cb = max(1, min(tile_items * ks, nu // 64))
    per_xcd_bound = (-(-nu // cb) + 7) // 8 * cb
    nx = max((ncu + 7) // 8, -(-per_xcd_bound // ST_MAX_ITEMS))
    share = (-(-n // cb) + 7) // 8 * cb
    return -(-share // nx) * -(-KB // ks)


@pytest.mark.parametrize("shape", [(2048, 512, 10, 512, 512), (4096, 128, 8, 1536, 1536),
                                   (2048, 64, 6, 1408, 5632)],
                         ids=lambda s: "x".join(map(str, s)))
def test_qwen_decode_gate_up_split_fewest_dealt_steps(shape, monkeypatch):
    """The Qwen decode K splits. Gate/up: of 1..min(KB / 4, 8) slices, the one
    whose busiest workgroup streams the fewest K steps under the launch's
    own deal, counting the tiles a uniform routing touches
    (E (1 - (1 - 1/E)^N) experts) and four steps per split; batches of 768
    bound items or more unsplit. C3 (the first shape): 4 / 2 / 1 / 4 / 4 / 1
    slices at 1 / 2 / 4 / 8 / 16 / 32 tokens. Down: the same deal, one step
    per item beyond its own, no finish charge, for the same batches; larger
    ones take the count-based split."""
    import math
    lib = _need_lib()
    H, E, k, I, Is = shape
    KB, slabs = H // 128, I // 128
    got = {}
    for T in (1, 2, 3, 4, 6, 8, 12, 16, 24, 32, 64):
        p = _plan(lib, 0, T, H, E, I, Is, k)
        if p[9] != 256:
            pytest.skip("port written for 256 CUs")
        N, bm, rt = T * k, p[1], p[3]
        sh_rt = -(-T // p[2])
        upper = rt * slabs + sh_rt * (Is // 128)
        touched = E * (1.0 - (1.0 - 1.0 / E) ** N)
        exp_rt = min(rt, math.ceil(touched + max(0.0, N - touched) / bm))
        exp = exp_rt * slabs + sh_rt * (Is // 128)
        want = 1
        if upper < 768:
            best = _dealt_steps(exp, upper, slabs, KB, 1)
            for ks in range(2, max(1, min(KB // 4, 8)) + 1):
                c = _dealt_steps(exp, upper, slabs, KB, ks) + 4
                if c < best:
                    want, best = ks, c
        assert p[5] == want and p[6] == want, (T, p[5], p[6], want)
        got[T] = p[5]
        # down: (steps + 1) per item, no finish charge, up to min(KB, 32)
        kbd = min(I, Is) // 128
        dn_up, dn_exp = rt * (H // 256) + sh_rt * (H // 256), exp_rt * (H // 256) + sh_rt * (H // 256)

        def dn_cost(ks):
            return (_dealt_steps(dn_exp, dn_up, H // 256, 1, ks) * (-(-kbd // ks) + 1))
        if upper < 768:
            want_dn = 1
            best = dn_cost(1)
            for ks in range(2, min(kbd, 32) + 1):
                if dn_cost(ks) < best:
                    want_dn, best = ks, dn_cost(ks)
        else:  # larger batches: the count-based rule
            monkeypatch.setenv("SLLM_MOE_SPLIT_DEALT", "0")
            want_dn = _plan(lib, 0, T, H, E, I, Is, k)[7]
            monkeypatch.delenv("SLLM_MOE_SPLIT_DEALT")
        assert p[7] == want_dn and p[8] == want_dn, (T, p[7], p[8], want_dn)
    if shape[0] == 2048 and shape[1] == 512:
        assert [got[t] for t in (1, 2, 4, 8, 16, 32)] == [4, 2, 1, 4, 4, 1]
