"""Pins the oracle's restatement of spec.py and splitkv_plan.py (CPU only)."""
import pytest

from oracle import plan as P


def test_spec_fixture():
    # tests/test_reference.py:60-65 of the reference.
    assert P.spec_values(32, 32, 8, 128, 8192) == (8, 32, 32 * 32 * 8 * 130 * 4)


@pytest.mark.parametrize("batch,heads,kv,capacity,splits,tokens", [
    (8, 8, 2, 1024, 8, 128), (8, 16, 4, 1024, 6, 192),
    (1, 16, 4, 2176, 36, 64), (1, 8, 2, 2176, 36, 64), (32, 32, 8, 8192, 1, 8192)])
def test_reference_plan_fixtures(batch, heads, kv, capacity, splits, tokens):
    # tests/test_splitkv_plan.py:7-13 of the reference (sm_count=108, D=256).
    plan = P.make_plan(batch, heads, kv, 256, capacity, 108)
    assert (plan["splits"], plan["tokens_per_split"]) == (splits, tokens)
    assert plan["table_capacity_tokens"] == (capacity + 255) // 256 * 256


def test_reference_explicit_fixture():
    plan = P.make_plan(1, 16, 4, 256, 2176, 108, num_splits=3)
    assert plan["splits"] == 3 and plan["tokens_per_split"] == 768 and plan["policy"] == "explicit"


@pytest.mark.parametrize("count", [-1, 129, 1.5])
def test_reference_bad_counts(count):
    with pytest.raises(ValueError, match="num_splits"):
        P.make_plan(1, 8, 2, 256, 1024, 108, num_splits=count)


def test_reference_bad_group():
    with pytest.raises(ValueError, match="16"):
        P.make_plan(1, 32, 1, 256, 1024, 108)


@pytest.mark.parametrize("args,expected", [
    # Hand derivations at sm_count=256 (virtual SMs 512).
    # B=1, Hkv=4, D=256, width 9 -> 36 blocks of 64; eff(n) = 4n/512 is
    # maximal at n=36 and the first eligible n reaching .85 of it is 36.
    ((1, 16, 4, 256, 2064, 256), (36, 64, 32)),
    ((1, 16, 4, 256, 2112, 256), (36, 64, 32)),
    # ctx 528 -> width 3, 12 blocks; eff maximal at the last eligible n=12.
    ((1, 16, 4, 256, 528, 256), (12, 64, 16)),
    # B=4, Hkv=2, D=128 (tile 128), width 4 -> 8 blocks -> 8 splits of 128.
    ((4, 8, 2, 128, 1000, 256), (8, 128, 8)),
    # B=64, Hkv=8: work = 64*8 = 512 >= f32(.8*512) -> 1 split.
    ((64, 32, 8, 128, 32768, 256), (1, 32768, 1)),
    # B=128 with Hkv 16 or 4: work 128*16 and 128*4 are >= 409.6 -> 1 split.
    ((128, 16, 16, 64, 4096, 256), (1, 4096, 1)),
    ((128, 32, 4, 256, 4096, 256), (1, 4096, 1)),
    # Rounding point: sm_count=5 -> vsm=10; f32(f32(.8)*10) == 8.0 exactly, so
    # work=8 takes one split.  Without the outer rounding 8 < 8.0000001 and the
    # heuristic would pick 5 (eff(5) = 4/4 = 1).
    ((8, 8, 1, 256, 2048, 5), (1, 2048, 1)),
    # work=7, vsm=10, 32 blocks, eligible n = 1..8: eff = .7,.7,.7, f32(2.8)/3,
    # 3.5/4, 4.2/5, 4.9/5, 5.6/6 -> best .98 (n=7); the first n with
    # eff >= .85*.98 = .833 is n=4 (.9333) -> 4 splits of 8 blocks = 512 tokens.
    ((7, 7, 1, 256, 2048, 5), (4, 512, 4)),
])
def test_hand_derived_plans(args, expected):
    plan = P.make_plan(*args)
    assert (plan["splits"], plan["tokens_per_split"], plan["lse_lanes"]) == expected
