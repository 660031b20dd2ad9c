"""Pins the oracle's restatement of the reference CPU path and fixed-1024 kernels.

The cases, lengths, geometries and tolerances are the reference's own
(tests/test_reference.py:8-81, examples/cpu_attention.py:9-20).
"""
import numpy as np
import pytest

from cases import make_case
from oracle import reference as R
from oracle import splitk as S
from oracle.numerics import bf16_round


def _fp32_case(lengths, hq=4, hkv=1, dim=64, seed=9, capacity=None):
    return make_case(lengths, hq, hkv, dim, seed, capacity, bf16=False)


@pytest.mark.parametrize("length", [0, 1, 255, 256, 257, 1023, 1024, 1025, 2051])
@pytest.mark.parametrize("dim,hq,hkv", [(64, 4, 1), (128, 4, 2), (64, 2, 2), (256, 8, 2)])
def test_streaming_and_split_match_independent_dense(length, dim, hq, hkv):
    args = _fp32_case([length, 1], hq, hkv, dim)
    expected = R.dense_reference(*args)
    for split in (False, True):
        actual = R.streaming_reference(*args, split=split)
        np.testing.assert_allclose(actual, expected, atol=3e-6, rtol=3e-5)
        assert np.isfinite(actual).all()


def test_dense_matches_float64_softmax():
    q, k, v, table, lengths = _fp32_case([700, 1, 0], 8, 2, 128, seed=3)
    out = R.dense_reference(q, k, v, table, lengths)
    for b, n in enumerate(lengths):
        if n == 0:
            assert not out[b].any()
            continue
        pos = np.arange(n)
        keys = k[table[b, pos // 256], pos % 256].astype(np.float64)
        vals = v[table[b, pos // 256], pos % 256].astype(np.float64)
        for h in range(8):
            s = keys[:, h // 4] @ q[b, h].astype(np.float64) / np.sqrt(128.0)
            w = np.exp(s - s.max())
            np.testing.assert_allclose(out[b, h], (w / w.sum()) @ vals[:, h // 4], atol=2e-6, rtol=1e-5)


def test_partial_page_poison_and_padding_are_ignored():
    args = list(_fp32_case([257, 0], capacity=1025))
    table = args[3]
    args[1][table[0, 1], 1:] = np.nan
    args[2][table[0, 1], 1:] = np.nan
    table[0, 2:] = -1
    table[1] = -1
    expected = R.dense_reference(*args)
    for split in (False, True):
        actual = R.streaming_reference(*args, split=split)
        np.testing.assert_allclose(actual, expected, atol=3e-6, rtol=3e-5)
        assert not actual[1].any()


def test_large_logits_stable_softmax():
    args = list(_fp32_case([1025], seed=23))
    args[0] *= 80
    args[1] *= 80
    expected = R.dense_reference(*args)
    np.testing.assert_allclose(R.streaming_reference(*args, split=True), expected, atol=1e-4)


@pytest.mark.parametrize("length,table", [(-1, [[0]]), (257, [[0]]), (1, [[-1]]), (1, [[2]])])
def test_invalid_metadata_rejected(length, table):
    with pytest.raises(ValueError):
        R.validate_metadata(np.array(table), np.array([length]), 2, 256)


def test_merge_of_nothing_is_zero():
    np.testing.assert_array_equal(R.merge_partials([], 64), np.zeros(64))


def test_cpu_attention_example_known_answer():
    # examples/cpu_attention.py:9-20: seed 7, table [[2,0,1]], length 257.
    rng = np.random.default_rng(7)
    q = rng.standard_normal((1, 4, 64)).astype(np.float32)
    k = rng.standard_normal((3, 256, 2, 64)).astype(np.float32)
    v = rng.standard_normal(k.shape).astype(np.float32)
    table = np.array([[2, 0, 1]], dtype=np.int32)
    lengths = np.array([257], dtype=np.int32)
    expected = R.dense_reference(q, k, v, table, lengths)
    actual = R.streaming_reference(q, k, v, table, lengths)
    assert np.allclose(actual, expected, atol=2e-5, rtol=2e-5)
    # Logical token 256 lives in physical page table[0, 1] = 0, slot 0.
    assert int(table[0, 256 // 256]) == 0 and 256 % 256 == 0
    # The reference reports max abs error ~1.0431e-7 (docs/VALIDATION.md:15).
    assert float(np.max(np.abs(actual - expected))) < 1e-6
    np.testing.assert_array_equal(R.gather_kv(k, table[0], 257)[256], k[0, 0])


@pytest.mark.parametrize("lengths,dim,hq,hkv", [
    ([0, 1, 255, 256, 257, 1023, 1024, 1025], 64, 4, 1),
    ([2051, 1, 0, 2049], 128, 4, 2),
    ([1025, 3000], 256, 8, 2)])
def test_fixed_kernels_match_streaming_reference(lengths, dim, hq, hkv):
    """_base == streaming (split=False) and _split+_merge == streaming (split=True),
    compared before the bf16 store at the reference's fp32 tolerance."""
    q, k, v, table, lens = make_case(lengths, hq, hkv, dim, capacity=max(lengths))
    base = S.base_decode(q, k, v, table, lens)
    stream = R.streaming_reference(q, k, v, table, lens)
    np.testing.assert_allclose(base, bf16_round(stream), atol=2e-6, rtol=8e-3)
    parts = -(-max(lengths) // 1024)
    ml = S.split_partitions(q, k, v, table, lens, parts)
    merged = S.ml_merge(*ml)
    split = R.streaming_reference(q, k, v, table, lens, split=True)
    np.testing.assert_allclose(merged, bf16_round(split), atol=2e-6, rtol=8e-3)
    for b, n in enumerate(lengths):
        if n == 0:
            assert not base[b].any() and not merged[b].any()
            assert np.all(ml[0][b] == -np.inf) and not ml[1][b].any()
