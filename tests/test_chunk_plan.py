"""The small-batch chunk planner of the base and fixed-split protocols (host code).

pd_plan_chunks cuts the table width of a batch whose walks (one workgroup per kv head
group and sequence, counted for the batch rounded up to a power of two) are fewer than
half the CUs into partitions of one workgroup each; pd_chunk_rows bounds the workspace
that serves every batch and width.  Checked against an independent restatement of the
rule, its invariants, and the benchmark shapes.
"""
import itertools

import pytest
import torch

from paged_decode import _native
from paged_decode.runtime import Resources, _chunk_plan
from paged_decode.spec import DecodeSpec


def walks_per_sequence(hq, hkv, dim):
    """Workgroups per sequence of the walk: kv heads in groups of 4 or 2 at D 64 when
    their query heads fit 16, else one per kv head and 16-head slice."""
    g = hq // hkv
    heads = 1
    if dim == 64:
        heads = 4 if hkv % 4 == 0 and 4 * g <= 16 else (2 if hkv % 2 == 0 and 2 * g <= 16 else 1)
    return hkv // heads if heads > 1 else hkv * -(-g // 16)


def restated(batch, hq, hkv, dim, width, sm):
    tile = 16384 // dim
    tiles = -(-width * 256 // tile)
    rounded = 1 << (batch - 1).bit_length()
    want = min(sm // (rounded * walks_per_sequence(hq, hkv, dim)), 128, tiles)
    if want < 2:
        return 1, width * 256
    per = -(-tiles // want)
    return -(-tiles // per), per * tile


GEOMETRIES = [(16, 4, 256), (32, 8, 128), (16, 16, 64), (8, 2, 256), (4, 1, 64), (40, 2, 256),
              (12, 4, 64), (6, 6, 64), (32, 1, 128), (64, 2, 128), (2, 2, 64)]


@pytest.mark.parametrize("hq,hkv,dim", GEOMETRIES)
def test_plan_matches_the_rule_and_its_invariants(hq, hkv, dim):
    tile = 16384 // dim
    for batch, width, sm in itertools.product((1, 2, 3, 5, 8, 17, 32, 64, 128, 300),
                                              (1, 2, 5, 9, 16, 33, 128, 513),
                                              (8, 80, 256, 304)):
        chunks, tokens = _native.plan_chunks(batch, hq, hkv, dim, width, sm)
        assert (chunks, tokens) == restated(batch, hq, hkv, dim, width, sm)
        walks = (1 << (batch - 1).bit_length()) * walks_per_sequence(hq, hkv, dim)
        if chunks == 1:
            assert tokens == width * 256
            continue
        assert 2 * walks <= sm and chunks <= min(128, sm // walks)
        # Padding the batch up to its next power of two keeps the plan.
        assert _native.plan_chunks(1 << (batch - 1).bit_length(), hq, hkv, dim, width,
                                   sm) == (chunks, tokens)
        assert tokens % tile == 0
        # The chunks cover the table, and none lies wholly past it.
        assert chunks * tokens >= width * 256 > (chunks - 1) * tokens
        assert batch * hq * chunks <= _native.chunk_rows(batch, hq, hkv, dim, sm)


def test_benchmark_shapes():
    # D256 GQA 16/4, capacity 2112 (9 pages): one 64-token tile per chunk at B=1.
    assert _native.plan_chunks(1, 16, 4, 256, 9, 256) == (36, 64)
    assert _native.plan_chunks(8, 16, 4, 256, 9, 256) == (8, 320)
    assert _native.plan_chunks(3, 16, 4, 256, 9, 256) == (12, 192)   # planned as 4
    # D128 GQA 32/8, capacity 4096.
    assert _native.plan_chunks(1, 32, 8, 128, 16, 256) == (32, 128)
    assert _native.plan_chunks(8, 32, 8, 128, 16, 256) == (4, 1024)
    # The bandwidth-sweep and edge-coverage batches fill the CUs: no chunks.
    assert _native.plan_chunks(64, 32, 8, 128, 128, 256) == (1, 32768)
    assert _native.plan_chunks(128, 16, 16, 64, 16, 256) == (1, 4096)
    assert _native.plan_chunks(128, 32, 4, 256, 16, 256) == (1, 4096)
    # The end-to-end decoder's full-attention layers (Hq 8, Hkv 2, D 256), B=1.
    assert _native.plan_chunks(1, 8, 2, 256, 9, 256) == (36, 64)


def test_chunk_rows_bounds_every_batch_and_width():
    for hq, hkv, dim in GEOMETRIES:
        for max_batch in (1, 4, 40, 200):
            rows = _native.chunk_rows(max_batch, hq, hkv, dim, 256)
            best = 0
            for batch in range(1, max_batch + 1):
                for width in range(1, 140):
                    chunks, _ = _native.plan_chunks(batch, hq, hkv, dim, width, 256)
                    if chunks > 1:
                        best = max(best, batch * hq * chunks)
            assert best <= rows
            # Tight: the bound is reached at a wide enough table.
            assert best == rows


def test_invalid_arguments_are_rejected():
    with pytest.raises(ValueError, match="head_dim"):
        _native.plan_chunks(1, 4, 1, 96, 4, 256)
    with pytest.raises(ValueError, match="divisible"):
        _native.plan_chunks(1, 5, 2, 64, 4, 256)
    with pytest.raises(ValueError, match="width"):
        _native.plan_chunks(1, 4, 1, 64, 0, 256)
    with pytest.raises(ValueError, match="SM"):
        _native.plan_chunks(1, 4, 1, 64, 4, 0)
    with pytest.raises(ValueError, match="positive"):
        _native.chunk_rows(0, 4, 1, 64, 256)


def _resources(spec, rows, sm):
    out = torch.empty((spec.max_batch, spec.num_heads, spec.head_dim), dtype=torch.bfloat16)
    return Resources(spec, out, chunk_maxima=torch.empty(rows), chunk_denoms=torch.empty(rows),
                     chunk_accums=torch.empty(rows * spec.head_dim), sm_count=sm)


def test_paged_decode_takes_the_chunks_only_with_a_large_enough_workspace():
    spec = DecodeSpec(8, 16, 4, 256, 2112)
    rows = _native.chunk_rows(8, 16, 4, 256, 256)
    res = _resources(spec, rows, 256)
    assert _chunk_plan(res, 1, 9) == (36, 64)
    assert _chunk_plan(res, 8, 9) == (8, 320)
    # A narrower live table runs the capacity plan's chunks that cover it.
    assert _chunk_plan(res, 1, 3) == (12, 64)
    assert _chunk_plan(res, 8, 1) == (1, 320)
    assert _chunk_plan(res, 7, 2) == (2, 320)
    # Without a workspace, or with one too small, every call walks.
    assert _chunk_plan(Resources(spec, res.out, sm_count=256), 1, 9) is None
    assert _chunk_plan(_resources(spec, 16 * 36 - 1, 256), 1, 9) is None
    # A batch that fills the CUs walks.
    assert _chunk_plan(_resources(DecodeSpec(64, 16, 4, 256, 2112), 4096, 256), 64, 9) is None
