"""Pins the oracle's KV-cache writes (CPU only)."""
import numpy as np

from oracle import kvwrite as KW


def test_write_pages_hand_example_crosses_a_page():
    # hybrid.py:66: physical = tables[:, pos // 256] * 256 + pos % 256.
    hkv, d = 1, 8
    k_pages = np.zeros((3, 256, hkv, d), np.float32)
    v_pages = np.zeros_like(k_pages)
    tables = np.array([[2, 0]], np.int32)
    positions = np.array([254, 255, 256, 257])
    key = np.arange(4 * d, dtype=np.float32).reshape(1, hkv, 4, d) + 1
    KW.write_pages(key, -key, k_pages, v_pages, tables, positions)
    assert (k_pages[2, 254, 0] == key[0, 0, 0]).all() and (k_pages[2, 255, 0] == key[0, 0, 1]).all()
    assert (k_pages[0, 0, 0] == key[0, 0, 2]).all() and (k_pages[0, 1, 0] == key[0, 0, 3]).all()
    assert (v_pages[0, 1, 0] == -key[0, 0, 3]).all()
    assert np.count_nonzero(k_pages) == 4 * d          # nothing else touched


def test_store_kvcache_skips_minus_one_and_matches_loops():
    rng = np.random.default_rng(0)
    n, hkv, d, slots = 9, 2, 4, 40
    key = rng.integers(1, 100, (n, hkv, d)).astype(np.int16)
    value = -key
    slot_mapping = rng.permutation(slots)[:n].astype(np.int32)
    slot_mapping[[2, 5]] = -1
    k_cache = np.zeros((slots // 8, 8, hkv, d), np.int16)
    v_cache = np.zeros_like(k_cache)
    KW.store_kvcache(key, value, k_cache, v_cache, slot_mapping)
    flat = k_cache.reshape(slots, hkv, d)
    for i, s in enumerate(slot_mapping):
        if s >= 0:
            assert (flat[s] == key[i]).all() and (v_cache.reshape(slots, hkv, d)[s] == value[i]).all()
    assert np.count_nonzero(flat.any(axis=(1, 2))) == n - 2


def test_the_two_write_forms_agree():
    # write_pages(B, Hkv, S, D) equals store_kvcache with the slot mapping the
    # nano-vLLM model runner builds (block_table[pos // 256] * 256 + pos % 256).
    rng = np.random.default_rng(1)
    b, hkv, steps, d, width = 2, 2, 300, 8, 3
    tables = rng.permutation(b * width).reshape(b, width).astype(np.int32)
    positions = np.arange(200, 200 + steps)
    key = rng.normal(size=(b, hkv, steps, d)).astype(np.float32)
    value = rng.normal(size=key.shape).astype(np.float32)
    k1 = np.zeros((b * width, 256, hkv, d), np.float32)
    v1 = np.zeros_like(k1)
    KW.write_pages(key, value, k1, v1, tables, positions)
    k2, v2 = np.zeros_like(k1), np.zeros_like(v1)
    slots = np.array([[tables[i, p // 256] * 256 + p % 256 for p in positions] for i in range(b)],
                     np.int32).reshape(-1)
    KW.store_kvcache(key.transpose(0, 2, 1, 3).reshape(-1, hkv, d),
                     value.transpose(0, 2, 1, 3).reshape(-1, hkv, d), k2, v2, slots)
    assert (k1 == k2).all() and (v1 == v2).all()
