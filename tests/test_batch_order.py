"""Rank arithmetic of the batch order (ordered_sequence in pd_device.h), on the CPU.

The multi-tile kernels hand grid row z to the sequence of length rank order_rank(z, B,
order), ranks ordering lengths decreasing with ties by increasing index.  These checks
restate that index arithmetic on integers and check the properties it is for: every
mapping is a permutation of the batch (no sequence skipped or served twice), rows that
share a CU (z and z + H) get ranks that sum to 2H - 1 (one long, one short), rows alone
on a CU get the longest sequences, and the rank rule agrees with a stable sort.  On the
GPU, tests/test_gpu_order.py checks that every output row is bit-identical to the same
sequence run alone.
"""
import numpy as np
import pytest


def order_rank(z, batch, order):
    if order <= 0 or batch > 2 * order:
        return z
    h = order
    paired = max(batch - h, 0)
    if z >= h:
        return batch - 1 - (z - h)
    return z - paired if z >= paired else h - paired + z


def ranks(lengths):
    """rank of sequence t: sequences longer, or as long with a smaller index."""
    n = len(lengths)
    return [sum(1 for u in range(n) if lengths[u] > lengths[t]
                or (lengths[u] == lengths[t] and u < t)) for t in range(n)]


@pytest.mark.parametrize("batch", [2, 3, 5, 16, 40, 48, 64, 100, 128, 255, 256])
def test_every_order_is_a_permutation(batch):
    for order in sorted({-1, 0, 1, 2, (batch + 1) // 2, batch // 2 + 3, batch, 2 * batch}):
        got = sorted(order_rank(z, batch, order) for z in range(batch))
        assert got == list(range(batch)), (batch, order)


@pytest.mark.parametrize("batch,h", [(64, 32), (48, 32), (40, 32), (128, 64), (33, 32),
                                     (7, 4), (256, 128)])
def test_cu_partners_get_one_long_and_one_short_sequence(batch, h):
    paired = batch - h
    for z in range(paired):
        assert order_rank(z, batch, h) + order_rank(z + h, batch, h) == 2 * h - 1
    alone = sorted(order_rank(z, batch, h) for z in range(paired, h))
    assert alone == list(range(h - paired))            # the longest sequences


def test_ranks_follow_a_stable_sort_by_decreasing_length():
    rng = np.random.default_rng(3)
    for batch in (2, 17, 64, 256):
        lengths = rng.integers(0, 6, size=batch)      # many ties
        r = ranks(lengths.tolist())
        order = np.argsort(-lengths, kind="stable")
        assert [int(order[k]) for k in range(batch)] == [r.index(k) for k in range(batch)]
        assert sorted(r) == list(range(batch))
