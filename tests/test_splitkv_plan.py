"""Native planner (pd_make_plan through make_splitkv_plan) vs reference fixtures and the oracle."""
import itertools

import pytest

from oracle import plan as oracle_plan
from paged_decode.spec import DecodeSpec
from paged_decode.splitkv_plan import make_splitkv_plan


@pytest.mark.parametrize("batch,heads,kv,capacity,splits,tokens", [
    (8, 8, 2, 1024, 8, 128), (8, 16, 4, 1024, 6, 192),
    (1, 16, 4, 2176, 36, 64), (1, 8, 2, 2176, 36, 64), (32, 32, 8, 8192, 1, 8192)])
def test_static_shape_examples(batch, heads, kv, capacity, splits, tokens):
    # tests/test_splitkv_plan.py:7-13 of the reference.
    plan = make_splitkv_plan(DecodeSpec(batch, heads, kv, 256, capacity), 108)
    assert (plan.splits, plan.tokens_per_split) == (splits, tokens)
    assert plan.table_capacity_tokens == (capacity + 255) // 256 * 256
    assert plan.policy == "pinned_geometry" and plan.sm_count == 108


def test_explicit_count_partitions_capacity_in_tiles():
    plan = make_splitkv_plan(DecodeSpec(1, 16, 4, 256, 2176), 108, num_splits=3)
    assert plan.splits == 3 and plan.tokens_per_split == 768
    assert plan.policy == "explicit"


@pytest.mark.parametrize("count", [-1, 129, 1.5, True])
def test_unsupported_explicit_counts(count):
    with pytest.raises(ValueError, match="num_splits"):
        make_splitkv_plan(DecodeSpec(1, 8, 2, 256, 1024), 108, num_splits=count)


@pytest.mark.parametrize("sm", [0, -3, 2.0, False])
def test_unsupported_sm_count(sm):
    with pytest.raises(ValueError, match="SM count"):
        make_splitkv_plan(DecodeSpec(1, 8, 2, 256, 1024), sm)


def test_unsupported_group():
    with pytest.raises(ValueError, match="16"):
        make_splitkv_plan(DecodeSpec(1, 32, 1, 256, 1024), 108)


def _as_dict(plan):
    return dict(splits=plan.splits, tile_tokens=plan.tile_tokens,
                tokens_per_split=plan.tokens_per_split,
                table_capacity_tokens=plan.table_capacity_tokens, lse_lanes=plan.lse_lanes,
                sm_count=plan.sm_count, policy=plan.policy)


def test_native_planner_matches_oracle_sweep():
    """Bit-exact agreement over a grid that includes the float32 rounding points."""
    checked = 0
    for batch, kv, group, dim, ctx, sm in itertools.product(
            (1, 2, 3, 4, 7, 8, 16, 64, 128), (1, 2, 4, 8), (1, 2, 4, 8, 16), (64, 128, 256),
            (1, 255, 528, 1000, 2064, 4096, 32768), (1, 5, 80, 104, 108, 132, 256, 304)):
        spec = DecodeSpec(batch, kv * group, kv, dim, ctx)
        for splits in (0, 3):
            native = _as_dict(make_splitkv_plan(spec, sm, num_splits=splits))
            expected = oracle_plan.make_plan(batch, kv * group, kv, dim, ctx, sm, splits)
            assert native == expected, (spec, sm, splits)
            checked += 1
    assert checked > 10000
