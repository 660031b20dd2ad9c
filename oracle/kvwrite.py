"""CPU restatement of the KV-cache writes (test infrastructure only).

store_kvcache: overlays/nano-vllm/nanovllm/layers/attention.py:10-38 (per token
i: slot = slot_mapping[i]; slot == -1 returns; cache row `slot` of
Hkv*D elements = key row i).  write_pages: src/paged_decode/hybrid.py:63-72
(physical = tables[:, pos // 256] * 256 + pos % 256; index_copy_ of
key.transpose(1, 2) rows into the pages viewed as [-1, Hkv, D]).
Arrays are modified in place, any dtype (uint16 bf16 bits in the tests).
"""
import numpy as np


def store_kvcache(key, value, k_cache, v_cache, slot_mapping):
    n = key.shape[0]
    kc = k_cache.reshape(-1, key.shape[1] * key.shape[2])
    vc = v_cache.reshape(-1, key.shape[1] * key.shape[2])
    for i in range(n):
        slot = int(slot_mapping[i])
        if slot == -1:
            continue
        kc[slot] = key[i].reshape(-1)
        vc[slot] = value[i].reshape(-1)


def write_pages(key, value, k_pages, v_pages, tables, positions):
    b, hkv, steps, d = key.shape
    physical = tables[:, positions // 256].astype(np.int64) * 256 + positions[None, :] % 256
    kp = k_pages.reshape(-1, hkv, d)
    vp = v_pages.reshape(-1, hkv, d)
    kp[physical.reshape(-1)] = key.transpose(0, 2, 1, 3).reshape(-1, hkv, d)
    vp[physical.reshape(-1)] = value.transpose(0, 2, 1, 3).reshape(-1, hkv, d)
