"""Static split-KV plan (mirrors splitkv_plan.py of the reference).

``make_splitkv_plan`` keeps the reference's signature, argument checks and
error messages (splitkv_plan.py:26-32) and computes the plan in the native
library (pd_make_plan, include/paged_decode.h), which reproduces the
reference's float32 rounding points exactly.
"""
from dataclasses import dataclass

from . import _native


@dataclass(frozen=True)
class SplitKVPlan:
    splits: int
    tile_tokens: int
    tokens_per_split: int
    table_capacity_tokens: int
    lse_lanes: int
    sm_count: int
    policy: str


def make_splitkv_plan(spec, sm_count, *, num_splits=0):
    if type(sm_count) is not int or sm_count < 1:
        raise ValueError("positive SM count required")
    if type(num_splits) is not int or not 0 <= num_splits <= 128:
        raise ValueError("num_splits must be an integer in [0,128]")
    if spec.num_heads // spec.num_kv_heads > 16:
        raise ValueError("matched split-KV requires at most 16 query heads per KV head")
    plan = _native.make_plan(spec.max_batch, spec.num_heads, spec.num_kv_heads, spec.head_dim,
                             spec.max_context_len, sm_count, num_splits)
    return SplitKVPlan(plan.splits, plan.tile_tokens, plan.tokens_per_split,
                       plan.table_capacity_tokens, plan.lse_lanes, plan.sm_count,
                       "explicit" if plan.is_explicit else "pinned_geometry")
