"""Restatement of the reference's base and fixed-1024 split-K kernels (test infrastructure).

Follows src/paged_decode/kernels.py of the reference repository:

* ``base_decode``      _base   kernels.py:10-41   one (b, h) online softmax, TILE=64,
                                                 natural exp, out = acc / denom (0 if denom == 0)
* ``split_partitions`` _split  kernels.py:44-80   same math per 1024-token partition,
                                                 storing unnormalized (m, l, acc)
* ``ml_merge``         _merge  kernels.py:83-100  M = max m (-inf -> 0), f = exp(m - M),
                                                 out = sum(acc f) / sum(l f) (total 0 -> 1)

All arithmetic is float32 as in the reference (K/V/Q widened to fp32,
kernels.py:21,24-25).  Outputs are rounded to bf16 (kernels.py:41,100 store fp32
into a bf16 tensor).  Pinned by tests/test_oracle_reference.py: these functions
agree with ``oracle.reference.streaming_reference`` (itself pinned to the
reference's test vectors) at the reference's fp32 tolerance, and with the dense
oracle; empty rows give exact zeros.
"""
import numpy as np

from .numerics import bf16_round
from .reference import gather_kv, PARTITION_SIZE, TILE_SIZE


def _online(qh, keys, vals, scale, tile=TILE_SIZE):
    # kernels.py:23-38 / 61-76: scores scaled before the max; natural exp.
    m = np.float32(-np.inf)
    l = np.float32(0)
    acc = np.zeros(qh.shape, dtype=np.float32)
    with np.errstate(invalid="ignore", over="ignore"):
        for start in range(0, len(keys), tile):
            s = (keys[start:start + tile] @ qh) * np.float32(scale)
            m_next = np.maximum(m, s.max())
            alpha = np.exp(np.float32(m - m_next))
            p = np.exp(s - m_next).astype(np.float32)
            acc = (acc * alpha + p @ vals[start:start + tile]).astype(np.float32)
            l = np.float32(l * alpha + p.sum())
            m = m_next
    return np.float32(m), np.float32(l), acc


def base_decode(q, k, v, table, lengths, scale=None):
    """_base: returns bf16-rounded [B, Hq, D] float32 array."""
    q = np.asarray(q, dtype=np.float32)
    scale = q.shape[-1] ** -0.5 if scale is None else scale
    B, Hq, D = q.shape
    group = Hq // k.shape[2]
    out = np.zeros((B, Hq, D), dtype=np.float32)
    for b in range(B):
        length = int(lengths[b])
        if length == 0:
            continue
        keys = gather_kv(k, table[b], length)
        vals = gather_kv(v, table[b], length)
        for h in range(Hq):
            _, l, acc = _online(q[b, h], keys[:, h // group], vals[:, h // group], scale)
            out[b, h] = acc / (l if l > 0 else np.float32(1))
    return bf16_round(out)


def split_partitions(q, k, v, table, lengths, partitions, scale=None, part_size=PARTITION_SIZE):
    """_split: (maxima, denoms, accums) with shapes [B,Hq,P], [B,Hq,P], [B,Hq,P,D]."""
    q = np.asarray(q, dtype=np.float32)
    scale = q.shape[-1] ** -0.5 if scale is None else scale
    B, Hq, D = q.shape
    group = Hq // k.shape[2]
    maxima = np.full((B, Hq, partitions), -np.inf, dtype=np.float32)
    denoms = np.zeros((B, Hq, partitions), dtype=np.float32)
    accums = np.zeros((B, Hq, partitions, D), dtype=np.float32)
    for b in range(B):
        length = int(lengths[b])
        keys = gather_kv(k, table[b], length)
        vals = gather_kv(v, table[b], length)
        for p in range(partitions):
            start = p * part_size
            if start >= length:       # kernels.py:62: empty partition keeps (-inf, 0, 0)
                continue
            end = min(start + part_size, length)
            for h in range(Hq):
                kv = h // group
                m, l, acc = _online(q[b, h], keys[start:end, kv], vals[start:end, kv], scale)
                maxima[b, h, p], denoms[b, h, p], accums[b, h, p] = m, l, acc
    return maxima, denoms, accums


def ml_merge(maxima, denoms, accums):
    """_merge: bf16-rounded [B, Hq, D] float32 array."""
    with np.errstate(invalid="ignore", over="ignore"):
        m_max = maxima.max(axis=-1, keepdims=True)
        m_max = np.where(m_max == -np.inf, np.float32(0), m_max).astype(np.float32)
        f = np.exp(maxima - m_max).astype(np.float32)
        total = (denoms * f).sum(axis=-1).astype(np.float32)
        num = (accums * f[..., None]).sum(axis=-2).astype(np.float32)
        out = num / np.where(total > 0, total, np.float32(1))[..., None]
    return bf16_round(out.astype(np.float32))
