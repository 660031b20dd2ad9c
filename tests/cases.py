"""Seeded synthetic inputs shared by the tests (NumPy side)."""
import numpy as np

from oracle.numerics import bf16_round


def make_case(lengths, hq=4, hkv=1, dim=64, seed=9, capacity=None, bf16=True):
    """Reference-style case (tests/test_reference.py:8-17 of the reference).

    default_rng(seed); the block table is a permutation of all physical pages;
    K, V, Q ~ N(0, 1).  With ``bf16`` the values are rounded to bf16 so the same
    arrays can be fed to the GPU operator unchanged.
    """
    rng = np.random.default_rng(seed)
    capacity = max(max(lengths), 1) if capacity is None else capacity
    pages_per_row = (capacity + 255) // 256
    pages = len(lengths) * pages_per_row
    table = rng.permutation(pages).reshape(len(lengths), pages_per_row).astype(np.int32)
    k = rng.normal(size=(pages, 256, hkv, dim)).astype(np.float32)
    v = rng.normal(size=k.shape).astype(np.float32)
    q = rng.normal(size=(len(lengths), hq, dim)).astype(np.float32)
    if bf16:
        q, k, v = bf16_round(q), bf16_round(k), bf16_round(v)
    return q, k, v, table, np.array(lengths, dtype=np.int32)


def poison_tails(k, v, table, lengths):
    """NaN-poison unused slots of each row's last live page and set dead table
    entries to -1, as tests/test_gpu.py:57-63 of the reference does."""
    for b, length in enumerate(lengths):
        length = int(length)
        live = (length + 255) // 256
        if length % 256:
            page = table[b, length // 256]
            k[page, length % 256:] = np.nan
            v[page, length % 256:] = np.nan
        table[b, live:] = -1
    return k, v, table
