"""Rank arithmetic of the batch order (ordered_sequence in pd_device.h), on the CPU.

When a multi-tile grid runs in two to four rounds (batch_order in pd_kernels.hip), grid
row z serves the sequence of length rank z, ranks ordering lengths decreasing with ties
by increasing index, so the longest items start first.  These checks restate that rank
rule on integers and check the properties it is for: the ranks are a permutation of the
batch (no sequence skipped or served twice) and agree with a stable sort.  On the GPU,
tests/test_gpu_order.py checks that every output row is bit-identical to the same
sequence run alone.
"""
import numpy as np


def ranks(lengths):
    """rank of sequence t: sequences longer, or as long with a smaller index."""
    n = len(lengths)
    return [sum(1 for u in range(n) if lengths[u] > lengths[t]
                or (lengths[u] == lengths[t] and u < t)) for t in range(n)]


def test_ranks_follow_a_stable_sort_by_decreasing_length():
    rng = np.random.default_rng(3)
    for batch in (2, 17, 64, 256):
        lengths = rng.integers(0, 6, size=batch)      # many ties
        r = ranks(lengths.tolist())
        order = np.argsort(-lengths, kind="stable")
        assert [int(order[k]) for k in range(batch)] == [r.index(k) for k in range(batch)]
        assert sorted(r) == list(range(batch))
