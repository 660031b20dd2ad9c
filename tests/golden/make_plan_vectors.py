"""Writes tests/golden/splitkv_plan_vectors.json: input/output vectors of the
reference's split-KV planner (src/paged_decode/splitkv_plan.py:26-56), run here
from the reference checkout to pin the planner restatements (oracle/plan.py and
the C++ pd_make_plan) beyond the reference's own fixtures, in particular at the
float32 rounding points of its efficiency heuristic for many CU counts.

Run in the development container only (the reference is not on GPU machines):
    python tests/golden/make_plan_vectors.py /root/reference
The fixture is data: [max_batch, num_heads, num_kv_heads, head_dim,
max_context_len, sm_count, num_splits] -> [splits, tile_tokens,
tokens_per_split, table_capacity_tokens, lse_lanes, policy] or an error string.
"""
import importlib.util
import json
import math
import os
import random
import sys
from types import SimpleNamespace


def load_planner(reference_root):
    path = os.path.join(reference_root, "src", "paged_decode", "splitkv_plan.py")
    spec = importlib.util.spec_from_file_location("_reference_splitkv_plan", path)
    module = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(module)
    return module.make_splitkv_plan


def cases(rng):
    sms = [1, 2, 3, 4, 5, 7, 8, 10, 13, 16, 32, 38, 64, 80, 104, 108, 110, 120, 128, 132,
           152, 228, 240, 256, 304]
    batches = [1, 2, 3, 4, 5, 6, 7, 8, 9, 12, 16, 24, 31, 32, 48, 64, 100, 128, 256]
    kvs = [1, 2, 3, 4, 5, 8, 16]
    groups = [1, 2, 4, 8, 16, 17]
    dims = [64, 128, 256]
    ctxs = [1, 64, 255, 256, 257, 511, 512, 528, 1000, 1024, 1025, 2048, 2051, 2064, 2112,
            2176, 4096, 8192, 16384, 32768, 65536, 131072]
    seen = set()
    # every CU count with the benchmark geometries, then a seeded sample
    fixed = [(1, 16, 4, 256, 2112), (1, 16, 4, 256, 528), (1, 16, 4, 256, 2064),
             (4, 8, 2, 128, 1000), (64, 32, 8, 128, 32768), (128, 16, 16, 64, 4096),
             (128, 32, 4, 256, 4096), (1, 8, 2, 256, 2112), (1, 16, 4, 256, 131072)]
    for sm in sms:
        for b, hq, hkv, d, ctx in fixed:
            for ns in (0, 1, 3, 6, 36):
                seen.add((b, hq, hkv, d, ctx, sm, ns))
    while len(seen) < 6000:
        hkv = rng.choice(kvs)
        key = (rng.choice(batches), hkv * rng.choice(groups), hkv, rng.choice(dims),
               rng.choice(ctxs), rng.choice(sms), rng.choice([0, 0, 0, 0, 1, 2, 7, 64, 128]))
        seen.add(key)
    return sorted(seen)


def main():
    reference = sys.argv[1] if len(sys.argv) > 1 else "/root/reference"
    make = load_planner(reference)
    rows = []
    for b, hq, hkv, d, ctx, sm, ns in cases(random.Random(20261202)):
        spec = SimpleNamespace(max_batch=b, num_heads=hq, num_kv_heads=hkv, head_dim=d,
                               max_context_len=ctx, table_width=math.ceil(ctx / 256))
        try:
            p = make(spec, sm, num_splits=ns)
            out = [p.splits, p.tile_tokens, p.tokens_per_split, p.table_capacity_tokens,
                   p.lse_lanes, p.policy]
        except ValueError as exc:
            out = "ValueError: " + str(exc)
        rows.append([[b, hq, hkv, d, ctx, sm, ns], out])
    target = os.path.join(os.path.dirname(os.path.abspath(__file__)), "splitkv_plan_vectors.json")
    with open(target, "w") as f:
        json.dump({"source": "src/paged_decode/splitkv_plan.py:26-56", "vectors": rows}, f,
                  separators=(",", ":"))
        f.write("\n")
    print(f"wrote {len(rows)} vectors to {target}")


if __name__ == "__main__":
    main()
