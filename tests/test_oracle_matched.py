"""Pins the oracle's restatement of the matched split-KV protocol (CPU only)."""
import types

import numpy as np
import pytest

import oracle.matched as M
from cases import make_case, poison_tails
from oracle import plan as P
from oracle import reference as R
from oracle.numerics import LOG2E, bf16_round, bf16_ulp_distance

# Output parity bar used throughout: at most one bf16 ulp apart, or an absolute
# difference below 1e-5 for values so close to zero that float32 accumulation
# noise exceeds their bf16 ulp.
ULP_FLOOR = 1e-5


def within_one_ulp(a, b):
    return (bf16_ulp_distance(a, b) <= 1) | (np.abs(a - b) <= ULP_FLOOR)


def run(case, plan):
    q, k, v, table, lengths = case
    return M.matched_decode(q, k, v, table, lengths, plan["splits"], plan["tokens_per_split"],
                            plan["tile_tokens"], plan["lse_lanes"])


GEOMETRIES = [
    # (lengths, hq, hkv, dim, capacity, num_splits)
    ([0, 1, 255, 256, 257, 1023, 1024, 1025], 8, 8, 256, 2051, 0),
    ([0, 1, 255, 256, 257, 1023, 1024, 1025], 8, 8, 256, 2051, 1),
    ([2064], 16, 4, 256, 2112, 0),
    ([528], 16, 4, 256, 528, 0),
    ([0, 1, 257, 1000], 8, 2, 128, 1000, 0),
    ([3000, 700, 4096], 8, 2, 128, 4096, 1),
    ([255, 1023, 2051], 4, 1, 64, 2051, 3),
    ([587, 587], 8, 2, 256, 1024, 6),
]


@pytest.mark.parametrize("lengths,hq,hkv,dim,cap,splits", GEOMETRIES)
def test_matches_independent_suffix_max_formulation(lengths, hq, hkv, dim, cap, splits):
    case = make_case(lengths, hq, hkv, dim, capacity=cap)
    plan = P.make_plan(len(lengths), hq, hkv, dim, cap, 256, num_splits=splits)
    out, _, _ = run(case, plan)
    independent = M.suffix_max_decode(*case, plan["splits"], plan["tokens_per_split"],
                                      plan["tile_tokens"])
    assert within_one_ulp(out, independent).all()
    dense = R.dense_reference(*case)
    np.testing.assert_allclose(out, dense, atol=2e-2, rtol=2e-2)


def test_error_magnitudes_match_reference_evidence():
    # evidence/correctness.json of the reference: D256, Hq=Hkv=8, lengths
    # [0,1,255,256,257,1023,1024,1025], capacity 2051, N(0,1) bf16 inputs:
    # max-abs 1.12e-3..1.41e-3 and RMSE 1.2e-4..1.52e-4 against the fp32 gather.
    case = make_case([0, 1, 255, 256, 257, 1023, 1024, 1025], 8, 8, 256, capacity=2051)
    plan = P.make_plan(8, 8, 8, 256, 2051, 108)
    out, _, _ = run(case, plan)
    err = np.abs(out - R.dense_reference(*case))
    assert 5e-4 < err.max() < 3e-3
    assert 7e-5 < np.sqrt((err ** 2).mean()) < 3e-4


def test_poisoned_tails_and_padding_never_read():
    lengths = [0, 1, 255, 256, 257, 1023, 1024, 2051]
    q, k, v, table, lens = make_case(lengths, 8, 2, 256, capacity=2051)
    clean = run((q, k, v, table, lens), P.make_plan(8, 8, 2, 256, 2051, 256, num_splits=6))[0]
    k, v, table = poison_tails(k.copy(), v.copy(), table.copy(), lens)
    out, partials, lse = run((q, k, v, table, lens), P.make_plan(8, 8, 2, 256, 2051, 256, num_splits=6))
    assert np.isfinite(out).all() and np.isfinite(partials).all()
    np.testing.assert_array_equal(out, clean)
    assert not out[0].any()
    assert np.all(lse[0] == -np.inf)


def test_single_live_partition_merge_returns_partial_exactly():
    case = make_case([100, 60], 4, 1, 128, capacity=1024)
    plan = P.make_plan(2, 4, 1, 128, 1024, 256, num_splits=4)    # 256 tokens per split
    out, partials, lse = run(case, plan)
    assert np.all(lse[:, :, 1:] == -np.inf)
    np.testing.assert_array_equal(out, bf16_round(partials[:, :, 0]))


def test_all_empty_rows_are_exact_zero():
    case = make_case([0, 0, 0], 8, 2, 64, capacity=2051)
    out, partials, lse = run(case, P.make_plan(3, 8, 2, 64, 2051, 256))
    assert not out.any() and not partials.any()
    assert np.all(lse == -np.inf)


def test_lse_is_log_sum_exp_of_scaled_scores():
    q, k, v, table, lens = make_case([1000, 77], 8, 2, 128, capacity=1024)
    plan = P.make_plan(2, 8, 2, 128, 1024, 256, num_splits=3)
    _, _, lse = run((q, k, v, table, lens), plan)
    T = plan["tokens_per_split"]
    for b, n in enumerate(lens):
        for p in range(plan["splits"]):
            start, end = p * T, min((p + 1) * T, int(n))
            if end <= start:
                assert np.all(lse[b, :, p] == -np.inf)
                continue
            pos = np.arange(start, end)
            keys = k[table[b, pos // 256], pos % 256].astype(np.float64)
            for h in range(8):
                s = keys[:, h // 4] @ q[b, h].astype(np.float64) * 128 ** -0.5
                ref = s.max() + np.log(np.exp(s - s.max()).sum())
                assert abs(lse[b, h, p] - ref) < 1e-5


def test_large_logits_stay_finite():
    q, k, v, table, lens = make_case([1025, 3], 4, 1, 64, seed=23, capacity=1025)
    case = (q * 80, k * 80, v, table, lens)
    plan = P.make_plan(2, 4, 1, 64, 1025, 256)
    out, _, _ = run(case, plan)
    assert np.isfinite(out).all()
    np.testing.assert_allclose(out, R.dense_reference(*case), atol=2e-2, rtol=2e-2)


def _mutant(old, new):
    src = open(M.__file__).read()
    assert old in src
    mod = types.ModuleType("oracle.matched_mutant")
    mod.__package__ = "oracle"
    exec(compile(src.replace(old, new), M.__file__, "exec"), mod.__dict__)
    return mod


@pytest.mark.parametrize("old,new", [
    ("t0 = start + (count - 1 - i) * tile", "t0 = start + i * tile"),           # forward walk
    ("np.matmul(bf16_round(p_[..., :nv])", "np.matmul((p_[..., :nv])"),         # no bf16(p)
    ("fma32(s, c, (-(m_next * c))[..., None])", "fma32(s, c, (-(m * c))[..., None])"),  # stale max
])
def test_planted_oracle_mistakes_are_caught(old, new):
    mutant = _mutant(old, new)
    case = make_case([3000, 700], 8, 2, 128, capacity=4096)
    plan = P.make_plan(2, 8, 2, 128, 4096, 256, num_splits=1)
    out, _, _ = mutant.matched_decode(*case, plan["splits"], plan["tokens_per_split"],
                                      plan["tile_tokens"], plan["lse_lanes"])
    independent = M.suffix_max_decode(*case, plan["splits"], plan["tokens_per_split"],
                                      plan["tile_tokens"])
    with np.errstate(invalid="ignore"):
        assert not within_one_ulp(out, independent).all()


@pytest.mark.parametrize("old,new", [
    ("t0 = start + (count - 1 - i) * tile", "t0 = start + i * tile"),
    ("np.matmul(bf16_round(p_[..., :nv])", "np.matmul((p_[..., :nv])"),
])
@pytest.mark.parametrize("lengths,hq,hkv,dim,cap,splits", [
    ([3000, 700], 8, 2, 128, 4096, 1), ([4096, 1000], 32, 4, 256, 4096, 1),
    ([1000, 2051], 8, 2, 128, 2051, 3)])
def test_parity_gate_rejects_protocol_mistakes(old, new, lengths, hq, hkv, dim, cap, splits):
    """The GPU parity gate (tests/parity.py) must fail a planted protocol mistake."""
    from parity import assert_parity
    mutant = _mutant(old, new)
    case = make_case(lengths, hq, hkv, dim, capacity=cap)
    plan = P.make_plan(len(lengths), hq, hkv, dim, cap, 256, num_splits=splits)
    args = (plan["splits"], plan["tokens_per_split"], plan["tile_tokens"], plan["lse_lanes"])
    wrong, _, _ = mutant.matched_decode(*case, *args)
    right, _, _, bound, _ = M.matched_decode_with_bounds(*case, *args)
    assert_parity(right, right, ambiguity=bound)
    with pytest.raises(AssertionError):
        assert_parity(wrong, right, ambiguity=bound)


@pytest.mark.parametrize("old,new", [
    # scores summed in float64 and rounded once (another summation order)
    ("s[..., :nv] = np.matmul(qb, kt.transpose(1, 2, 0))",
     "s[..., :nv] = np.matmul(qb.astype(np.float64), "
     "kt.transpose(1, 2, 0).astype(np.float64)).astype(F32)"),
    # exp2 evaluated in float64 and rounded once (another exp2 instruction)
    ("p_ = exp2_32(fma32(s, c, (-(m_next * c))[..., None]))",
     "p_ = np.exp2(fma32(s, c, (-(m_next * c))[..., None]).astype(np.float64)).astype(F32)"),
])
@pytest.mark.parametrize("seed", [1, 2])
def test_ambiguity_bound_covers_fp32_rounding_differences(old, new, seed):
    """Faithful implementations that only differ in fp32 rounding pass the gate,
    although individual near-zero outputs move by many bf16 ulps."""
    from parity import assert_parity
    variant = _mutant(old, new)
    case = make_case([4096, 4000, 1000, 2000, 3000, 256], 32, 4, 256, seed=seed, capacity=4096)
    plan = P.make_plan(6, 32, 4, 256, 4096, 256, num_splits=1)
    args = (plan["splits"], plan["tokens_per_split"], plan["tile_tokens"], plan["lse_lanes"])
    other, other_partials, _ = variant.matched_decode(*case, *args)
    right, partials, _, bound, partial_bound = M.matched_decode_with_bounds(*case, *args)
    assert_parity(other, right, ambiguity=bound)
    assert (np.abs(other_partials - partials) <= partial_bound + 2e-5 + 2e-5 * np.abs(partials)).all()


def test_scale_log2_constant():
    # SCALE_LOG2 = scale * 1.4426950408889634 in double, used as float32.
    assert LOG2E == 1.4426950408889634
    assert np.float32(256 ** -0.5 * LOG2E) == np.float32(0.09016844)
