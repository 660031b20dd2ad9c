"""Restatement of the reference's geometry contract and split-KV planner (test infrastructure).

* ``spec_values``  spec.py:32-42   partitions = ceil(ctx / 1024), table_width =
                                   ceil(ctx / 256), split workspace bytes
* ``make_plan``    splitkv_plan.py:26-56  (``_f32`` at :11-12)

The planner mixes Python float (double) arithmetic with explicit rounding to
float32 at exactly three places: f32(f32(.8) * virtual_sms) (:40),
waves = f32(f32(work * n) / virtual_sms) (:48) and eff = f32(waves / ceil(waves))
(:49); the ``.85 * best`` threshold (:51) is compared in double.  ``_f32`` here
uses ``struct`` float packing exactly like the reference.

Pinned by tests/test_oracle_plan.py: the reference's fixtures
(tests/test_splitkv_plan.py:7-30 at sm_count=108, explicit 3 splits -> 768
tokens, the error cases) and the spec fixture (tests/test_reference.py:60-65),
plus hand-derived known answers at float32 rounding points (for example
sm_count=5, work=8: f32(f32(.8)*10) rounds to exactly 8.0 so the plan is one
split, while an unrounded product would give five).
"""
import math
import struct

PAGE_SIZE = 256
PARTITION_SIZE = 1024


def _f32(value):
    return struct.unpack("f", struct.pack("f", value))[0]


def spec_values(max_batch, num_heads, num_kv_heads, head_dim, max_context_len):
    partitions = math.ceil(max_context_len / PARTITION_SIZE)
    width = math.ceil(max_context_len / PAGE_SIZE)
    workspace = max_batch * num_heads * partitions * (head_dim + 2) * 4
    return partitions, width, workspace


def make_plan(max_batch, num_heads, num_kv_heads, head_dim, max_context_len, sm_count,
              num_splits=0):
    """Returns a dict with the reference SplitKVPlan fields."""
    if type(sm_count) is not int or sm_count < 1:
        raise ValueError("positive SM count required")
    if type(num_splits) is not int or not 0 <= num_splits <= 128:
        raise ValueError("num_splits must be an integer in [0,128]")
    if num_heads // num_kv_heads > 16:
        raise ValueError("matched split-KV requires at most 16 query heads per KV head")
    tile = 256 if head_dim == 64 else (128 if head_dim == 128 else 64)
    width = math.ceil(max_context_len / PAGE_SIZE)
    capacity = width * 256
    blocks = (capacity + tile - 1) // tile
    splits = num_splits
    if not splits:
        work = max_batch * num_kv_heads
        vsm = sm_count * 2
        if work >= _f32(_f32(.8) * vsm):
            splits = 1
        else:
            top = min(128, vsm, blocks)
            eff = {}
            for n in range(1, top + 1):
                if n == 1 or math.ceil(blocks / n) != math.ceil(blocks / (n - 1)):
                    waves = _f32(_f32(work * n) / vsm)
                    eff[n] = _f32(waves / math.ceil(waves))
            best = max(eff.values())
            splits = next(n for n, e in eff.items() if e >= .85 * best)
    padded = 1 << (splits - 1).bit_length()
    merge_rows = 4 if head_dim % 128 == 0 else 8
    return dict(splits=splits, tile_tokens=tile,
                tokens_per_split=math.ceil(blocks / splits) * tile,
                table_capacity_tokens=capacity,
                lse_lanes=min(padded, 128 // merge_rows), sm_count=sm_count,
                policy="explicit" if num_splits else "pinned_geometry")
