"""Restatement of the reference's NumPy CPU path (test infrastructure).

Follows src/paged_decode/reference.py of the reference repository:

* ``validate_metadata``  reference.py:10-21
* ``gather_kv``          reference.py:24-28
* ``dense_reference``    reference.py:31-46   (independent dense softmax)
* ``partial``            reference.py:49-60   (tiled online softmax, TILE=64)
* ``merge_partials``     reference.py:63-71
* ``streaming_reference`` reference.py:74-88  (split mode: 1024-token partitions)

Pinned by tests/test_oracle_reference.py with the reference's own cases from
tests/test_reference.py:20-81 (streaming/split vs dense at the same lengths,
geometries and tolerances, NaN-poisoned tails, -1 padding, x80 logits, invalid
metadata) and the known answer of examples/cpu_attention.py (seed 7, table
[[2,0,1]], length 257).  ``dense_reference`` is additionally checked against a
float64 softmax written with different array operations.
"""
import numpy as np

PAGE_SIZE = 256          # spec.py:6
PARTITION_SIZE = 1024    # spec.py:7
TILE_SIZE = 64           # spec.py:8


def validate_metadata(table, lengths, num_pages, max_context_len, page_size=PAGE_SIZE):
    table, lengths = np.asarray(table), np.asarray(lengths)
    if table.ndim != 2 or lengths.ndim != 1 or len(table) != len(lengths):
        raise ValueError("metadata batch dimensions differ")
    if not (np.issubdtype(table.dtype, np.integer) and np.issubdtype(lengths.dtype, np.integer)):
        raise ValueError("metadata must be integral")
    if np.any(lengths < 0) or np.any(lengths > max_context_len):
        raise ValueError("context length outside configured capacity")
    for row, length in zip(table, lengths):
        live = (int(length) + page_size - 1) // page_size
        if live > len(row):
            raise ValueError("invalid live page mapping")
        pages = row[:live]
        if np.any(pages < 0) or np.any(pages >= num_pages):
            raise ValueError("invalid live page mapping")


def gather_kv(cache, table_row, length):
    """Logical rows 0..length-1 of one sequence: cache[table[t // 256], t % 256]."""
    if length == 0:
        return np.empty((0, *cache.shape[2:]), dtype=np.float32)
    pos = np.arange(length)
    page_size = cache.shape[1]
    return cache[np.asarray(table_row)[pos // page_size], pos % page_size].astype(np.float32)


def dense_reference(q, k, v, table, lengths, scale=None):
    """Independent FP32 oracle: full softmax over the gathered context per (b, h)."""
    q = np.asarray(q, dtype=np.float32)
    scale = q.shape[-1] ** -0.5 if scale is None else scale
    validate_metadata(table, lengths, len(k), table.shape[1] * k.shape[1], k.shape[1])
    out = np.zeros_like(q)
    group = q.shape[1] // k.shape[2]
    for b, length in enumerate(np.asarray(lengths)):
        length = int(length)
        if length == 0:
            continue
        keys = gather_kv(k, table[b], length)
        vals = gather_kv(v, table[b], length)
        for h in range(q.shape[1]):
            kv = h // group
            s = (keys[:, kv] @ q[b, h]) * np.float32(scale)
            w = np.exp(s - s.max())
            out[b, h] = (w @ vals[:, kv]) / w.sum()
    return out


def partial(q, keys, vals, scale, tile=TILE_SIZE):
    """Online softmax state (m, l, acc) over one run of keys, tile by tile."""
    m, l = np.float32(-np.inf), np.float32(0)
    acc = np.zeros(q.shape, dtype=np.float32)
    with np.errstate(invalid="ignore", over="ignore"):
        for start in range(0, len(keys), tile):
            s = (keys[start:start + tile] @ q) * np.float32(scale)
            m_next = np.maximum(m, s.max())
            alpha = np.exp(m - m_next)
            p = np.exp(s - m_next)
            acc = acc * alpha + p @ vals[start:start + tile]
            l = l * alpha + p.sum()
            m = m_next
    return m, l, acc


def merge_partials(parts, dim):
    """Merge (m, l, acc) states of disjoint runs; empty runs (l == 0) are dropped."""
    live = [(m, l, a) for m, l, a in parts if l > 0]
    if not live:
        return np.zeros(dim, dtype=np.float32)
    m = max(p[0] for p in live)
    factors = [np.exp(p[0] - m) for p in live]
    num = sum(f * p[2] for f, p in zip(factors, live))
    den = sum(f * p[1] for f, p in zip(factors, live))
    return num / den


def streaming_reference(q, k, v, table, lengths, split=False, scale=None):
    """Tiled online softmax; with ``split`` the context is cut into 1024-token partitions."""
    scale = q.shape[-1] ** -0.5 if scale is None else scale
    validate_metadata(table, lengths, len(k), table.shape[1] * k.shape[1], k.shape[1])
    out = np.zeros(q.shape, dtype=np.float32)
    group = q.shape[1] // k.shape[2]
    for b, length in enumerate(np.asarray(lengths)):
        length = int(length)
        keys = gather_kv(k, table[b], length)
        vals = gather_kv(v, table[b], length)
        for h in range(q.shape[1]):
            step = PARTITION_SIZE if split else max(1, length)
            kv = h // group
            qh = np.asarray(q[b, h], dtype=np.float32)
            parts = [partial(qh, keys[s:s + step, kv], vals[s:s + step, kv], scale)
                     for s in range(0, length, step)]
            out[b, h] = merge_partials(parts, q.shape[-1])
    return out
