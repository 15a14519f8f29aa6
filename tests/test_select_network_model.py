"""CPU model of the search kernel's register sorting networks (frnn_device.hpp:
bitonic_step / wave_sort_u64 / wave_bitonic_merge_u64, and the final
selections of search_kernel.hip: final_small, final_group).

A register holds one 64-bit key per lane of the 64-lane wave.  bitonic_step(k,
j) exchanges lane i with lane i ^ j; lane i keeps the minimum iff (bit j of i
is clear) == (bit k of the element index is clear), k = 0 meaning ascending
everywhere and k = 64 (a bit no lane index has) likewise.  The model replays
the same level/stage schedules on random keys with ties in the high word and
checks what the kernel relies on:

* the full 21-stage network sorts a register ascending;
* levels 1..L-1 plus a last level with k = 64 sort every block of 2^L lanes
  ascending (four lists of <= 16 keys, or two of <= 32, per register);
* the first four levels alone leave lanes 48..63 descending, so a second
  register of <= 16 keys there, behind ~0 fill, is descending over all 64
  lanes, and min(x0[i], x1[i]) with x0 ascending is bitonic and holds the 64
  smallest of both, which the six half-cleaner stages sort.
"""
import numpy as np
import pytest

W = 64
FILL = np.uint64(0xFFFFFFFFFFFFFFFF)


def step(x, k, j):
    lane = np.arange(W)
    p = x
    q = x[lane ^ j]
    up = np.ones(W, bool) if k in (0, W) else (lane & k) == 0
    keep_min = ((lane & j) == 0) == up
    return np.where((p < q) == keep_min, p, q)


def levels(x, first, last, last_k=None):
    for lk in range(first, last + 1):
        k = 1 << lk
        if lk == last and last_k is not None:
            k = last_k
        for lj in range(lk - 1, -1, -1):
            x = step(x, k, 1 << lj)
    return x


def merge(x):
    for lj in range(5, -1, -1):
        x = step(x, 0, 1 << lj)
    return x


def keys(rs, n):
    # high words from a small range (ties in d2), distinct low words (indices)
    hi = rs.randint(0, 8, n).astype(np.uint64)
    lo = rs.permutation(1 << 20)[:n].astype(np.uint64)
    return (hi << np.uint64(32)) | lo


def test_full_network_sorts_a_register():
    rs = np.random.RandomState(1)
    for _ in range(50):
        n = int(rs.randint(0, W + 1))
        x = np.full(W, FILL)
        x[:n] = keys(rs, n)
        y = levels(x, 1, 6)
        assert np.array_equal(y, np.sort(x))


@pytest.mark.parametrize("lw", [4, 5])
def test_grouped_lists_sort_per_block(lw):
    # final_group: 64 / 2^lw lists of <= 2^lw keys each, one per block
    rs = np.random.RandomState(2 + lw)
    blk = 1 << lw
    for _ in range(50):
        x = np.full(W, FILL)
        for g in range(W // blk):
            n = int(rs.randint(0, blk + 1))
            x[g * blk:g * blk + n] = keys(rs, n)
        y = levels(x, 1, lw, last_k=W)
        for g in range(W // blk):
            assert np.array_equal(y[g * blk:(g + 1) * blk], np.sort(x[g * blk:(g + 1) * blk]))


def test_partial_second_register_and_merge():
    # final_small: x0 holds 64 keys, x1 holds w <= 16 more in lanes 48..63
    rs = np.random.RandomState(3)
    for _ in range(100):
        w = int(rs.randint(1, 17))
        allk = keys(rs, W + w)
        x0 = levels(allk[:W].copy(), 1, 6)
        x1 = np.full(W, FILL)
        x1[W - 16:W - 16 + w] = allk[W:]
        x1 = levels(x1, 1, 4)
        assert np.all(np.diff(x1.astype(object)) <= 0)      # descending over all 64 lanes
        c = np.minimum(x0, x1)
        y = merge(c)
        assert np.array_equal(y, np.sort(allk)[:W])


def test_full_second_register_reversed():
    # final_small with w > 16: x1 sorted ascending and reversed
    rs = np.random.RandomState(4)
    for _ in range(50):
        w = int(rs.randint(17, W + 1))
        allk = keys(rs, W + w)
        x0 = levels(allk[:W].copy(), 1, 6)
        x1 = np.full(W, FILL)
        x1[:w] = allk[W:]
        x1 = levels(x1, 1, 6)[::-1]
        y = merge(np.minimum(x0, x1))
        assert np.array_equal(y, np.sort(allk)[:W])
