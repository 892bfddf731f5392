"""Expert-major token permutation (oracle side).

The canonical order of the T*k (token, slot) assignments is ascending
expert id, then ascending flat index t*k + j, i.e.
np.argsort(ids.ravel(), kind="stable"). Per-expert counts are the
bincount of the flat ids (ref/hf_sources/dsv4/model.py:689); the dispatch
that follows, torch.where(indices == i) (:693), visits the rows of expert
i in ascending token order, which is exactly this order restricted to i.

Pinned by tests/test_oracle_permute.py with a brute-force double loop over
experts and assignments.
"""

from __future__ import annotations

import numpy as np


def permute(ids, num_experts: int):
    """ids (T, k) integer expert ids -> dict with
    counts (E,) int32, offsets (E+1,) int32 (exclusive prefix sum),
    sorted_idx (T*k,) int32: flat assignment index t*k+j at each position,
    inv_pos (T*k,) int32: position of flat assignment t*k+j."""
    ids = np.asarray(ids)
    flat = ids.reshape(-1).astype(np.int64)
    if flat.size and (flat.min() < 0 or flat.max() >= num_experts):
        raise ValueError("expert id out of range")
    order = np.argsort(flat, kind="stable")
    counts = np.bincount(flat, minlength=num_experts).astype(np.int32)
    offsets = np.zeros(num_experts + 1, np.int32)
    np.cumsum(counts, out=offsets[1:])
    inv = np.empty_like(order)
    inv[order] = np.arange(order.size)
    return dict(counts=counts, offsets=offsets,
                sorted_idx=order.astype(np.int32), inv_pos=inv.astype(np.int32))
