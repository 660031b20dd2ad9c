"""The planner restatements against vectors of the reference planner itself.

tests/golden/splitkv_plan_vectors.json holds 6000 input/output vectors of
make_splitkv_plan (src/paged_decode/splitkv_plan.py:26-56), written by
tests/golden/make_plan_vectors.py from the reference checkout: the benchmark
geometries at 25 CU counts plus a seeded sample over batch, heads, group size,
head dim, context and explicit split counts, including the float32 rounding
points of the efficiency heuristic and the error cases.  Both the oracle and the
C++ planner of the library (pd_make_plan, host code) must reproduce every one.
"""
import json
import os

import pytest

from oracle import plan as P

HERE = os.path.dirname(os.path.abspath(__file__))


def _vectors():
    with open(os.path.join(HERE, "golden", "splitkv_plan_vectors.json")) as f:
        return json.load(f)["vectors"]


def test_oracle_matches_reference_vectors():
    mismatches = []
    for (b, hq, hkv, d, ctx, sm, ns), expected in _vectors():
        try:
            p = P.make_plan(b, hq, hkv, d, ctx, sm, num_splits=ns)
            got = [p["splits"], p["tile_tokens"], p["tokens_per_split"],
                   p["table_capacity_tokens"], p["lse_lanes"], p["policy"]]
        except ValueError as exc:
            got = "ValueError: " + str(exc)
        if got != expected:
            mismatches.append(((b, hq, hkv, d, ctx, sm, ns), got, expected))
    assert not mismatches, mismatches[:5]


def test_library_planner_matches_reference_vectors():
    from paged_decode.spec import DecodeSpec
    from paged_decode.splitkv_plan import make_splitkv_plan
    mismatches = []
    for (b, hq, hkv, d, ctx, sm, ns), expected in _vectors():
        try:
            p = make_splitkv_plan(DecodeSpec(b, hq, hkv, d, ctx), sm, num_splits=ns)
            got = [p.splits, p.tile_tokens, p.tokens_per_split, p.table_capacity_tokens,
                   p.lse_lanes, p.policy]
        except ValueError as exc:
            got = "ValueError: " + str(exc)
        if got != expected:
            mismatches.append(((b, hq, hkv, d, ctx, sm, ns), got, expected))
    assert not mismatches, mismatches[:5]
