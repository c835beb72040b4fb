"""The top-k kernel's threshold search (select.hip, kth_key) decides only the
bits below those that its lower bound and the row's largest key share.  This
CPU emulation of the wave-level select checks that the shortened search
selects the same set as the bit-by-bit search from bit 31 (the selection rule
of lcv_bsa_topk: the k largest scores, ties to the lower column, NaN below
-inf, -0.0 equal to +0.0) over rows with Gaussian scores, heavy ties, one
shared exponent, NaN and -0.0, and near-constant rows."""

from __future__ import annotations

import numpy as np
import pytest


def _order_key(f: np.ndarray) -> np.ndarray:
    u = f.astype(np.float32).view(np.uint32).astype(np.uint64)
    u = np.where(f == 0, 0, u)  # -0.0 -> +0.0
    k = np.where(u & 0x80000000, (~u) & 0xFFFFFFFF, u | 0x80000000)
    return np.where(np.isnan(f), 0, k).astype(np.uint64)


def _search(keys: np.ndarray, k: int, floor: int, start_bit: int, thr: int) -> int:
    for bit in range(start_bit, -1, -1):
        cand = thr | (1 << bit)
        cnt = int((keys >= cand).sum())
        if cnt >= k:
            thr = cand
            if cnt == k and cand >= floor:
                break
    return thr


def _full(keys, k, floor):
    return _search(keys, k, floor, 31, 0)


def _shortened(keys, k, floor, hi):
    diff = floor ^ hi
    if diff == 0:
        return floor
    top = diff.bit_length() - 1
    return _search(keys, k, floor, top, floor & ~((2 << top) - 1) & 0xFFFFFFFF)


def _selected(keys, thr, k):
    gt = np.flatnonzero(keys > thr)
    eq = np.flatnonzero(keys == thr)[: k - len(gt)]
    return sorted(np.concatenate([gt, eq]).tolist())


def _row(rng, mode, nk):
    if mode == 0:
        return rng.normal(size=nk).astype(np.float32)
    if mode == 1:
        return rng.integers(-3, 4, size=nk).astype(np.float32)
    if mode == 2:
        return (30 + rng.random(nk)).astype(np.float32)
    if mode == 3:
        sc = rng.normal(size=nk).astype(np.float32)
        sc[rng.integers(0, nk, 5)] = np.nan
        sc[rng.integers(0, nk, 5)] = -0.0
        return sc
    sc = np.full(nk, 2.5, np.float32)
    sc[rng.integers(0, nk, 3)] = 7.0
    return sc


@pytest.mark.parametrize("mode", range(5))
def test_shortened_search_selects_the_same_set(mode):
    rng = np.random.default_rng(100 + mode)
    checked = 0
    for _ in range(600):
        nk = int(rng.integers(64, 1025))
        k = int(rng.integers(1, 65))
        keys = _order_key(_row(rng, mode, nk))
        per = (nk + 63) // 64
        lanes = np.zeros(per * 64, np.uint64)
        lanes[:nk] = keys
        lanes = lanes.reshape(per, 64)  # register e of lane l holds column 64 e + l
        floor = int(lanes.max(axis=0).min())  # smallest of the lanes' largest keys
        hi = int(lanes.max())
        cand = keys[keys >= floor]  # the compacted candidates, in column order
        assert len(cand) >= 64 >= k
        t_full, t_short = _full(cand, k, floor), _shortened(cand, k, floor, hi)
        assert _selected(cand, t_full, k) == _selected(cand, t_short, k)
        checked += 1
    assert checked == 600


def test_shortened_search_fallback_is_the_full_search():
    """Without a bound (floor 0, hi all ones) the search starts at bit 31."""
    rng = np.random.default_rng(7)
    for _ in range(200):
        keys = _order_key(rng.normal(size=300).astype(np.float32))
        k = int(rng.integers(1, 300))
        assert _shortened(keys, k, 0, 0xFFFFFFFF) == _full(keys, k, 0)
