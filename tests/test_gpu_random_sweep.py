"""Seeded random sweep of the operator against the oracle, every backend.

Each case draws its geometry (D 64 / 128 / 256, 1-8 kv heads, 1-16 query heads
per kv head, up to 24 for the base and fixed-split protocols), a batch of 1-8
sequences with lengths mixing uniform draws and tile, page and capacity
boundaries, a table capacity up to 2600 tokens, NaN-poisoned tails and -1 table
padding, sometimes a custom softmax scale, and one backend:
* the matched protocol with the planner's plan, an explicit split count, or the
  single-launch (fused) merge, which must equal the two launches bit for bit;
* the base protocol (hip_base) and the fixed 1024-token protocol (hip_splitk),
  alternately through the walk (resources without the chunk workspace) and through
  whatever grid paged_decode picks (the small-batch chunks at these batches).
Every output passes the oracle's one-ulp gate and the dense 2e-2 gate; matched
LSEs match the oracle's.  Outputs and workspaces start NaN-poisoned.

A second sweep draws batches of 8-12 sequences with an explicit split count whose
workgroups outnumber the CUs in splits of 2 to 5 tiles, so that the partition walks
several splits per workgroup: outputs and LSEs must equal the single-launch path's
(one workgroup per split) bit for bit, and pass the oracle's gate.
"""
import numpy as np
import pytest
import torch

if not torch.cuda.is_available():
    pytest.skip("needs an MI355X GPU", allow_module_level=True)

from cases import make_case, poison_tails
from gpu_cases import (assert_close_dense, assert_within_one_ulp, poison_workspace, to_gpu,
                       to_np, torch_dense)
from oracle import matched as OM
from oracle import splitk as OS
from paged_decode.matched_splitkv import allocate_matched_resources, matched_decode
from paged_decode.runtime import allocate_resources, paged_decode
from paged_decode.spec import DecodeSpec

pytestmark = pytest.mark.gpu

BACKENDS = ("matched", "matched_splits", "matched_fused", "hip_base", "hip_splitk")
CASES = 180
BOUNDARIES = (0, 1, 2, 63, 64, 65, 127, 128, 129, 255, 256, 257, 511, 512, 513, 1023, 1024,
              1025)


def draw(index):
    rng = np.random.default_rng(5000 + index)
    backend = BACKENDS[index % len(BACKENDS)]
    dim = int(rng.choice([64, 128, 256]))
    hkv = int(rng.choice([1, 2, 3, 4, 6, 8]))
    groups = [1, 2, 3, 4, 5, 8, 12, 16] + ([20, 24] if backend.startswith("hip") else [])
    group = int(rng.choice(groups))
    while group * hkv > 64:
        group //= 2
    batch = int(rng.integers(1, 9))
    capacity = int(rng.integers(1, 2601))
    lengths = rng.integers(0, capacity + 1, size=batch)
    for b in range(batch):
        if rng.random() < 0.4:
            lengths[b] = min(int(rng.choice(BOUNDARIES + (capacity,))), capacity)
    scale = float(rng.uniform(0.02, 0.2)) if rng.random() < 0.25 else None
    tile = 16384 // dim
    blocks = -(-(-(-capacity // 256) * 256) // tile)
    splits = int(rng.integers(1, min(9, blocks) + 1))
    return dict(backend=backend, dim=dim, hq=group * hkv, hkv=hkv, batch=batch,
                capacity=capacity, lengths=[int(x) for x in lengths], scale=scale,
                splits=splits, seed=index)


@pytest.mark.parametrize("index", range(CASES))
def test_random_case(index):
    c = draw(index)
    where = f"case {index}: {c}"
    q, k, v, table, lens = make_case(c["lengths"], c["hq"], c["hkv"], c["dim"], seed=c["seed"],
                                     capacity=c["capacity"])
    poison_tails(k, v, table, lens)
    case = (q, k, v, table, lens)
    g = to_gpu(case)
    spec = DecodeSpec(c["batch"], c["hq"], c["hkv"], c["dim"], c["capacity"])
    scale = c["scale"]
    backend = c["backend"]
    if backend.startswith("matched"):
        res = allocate_matched_resources(spec, "cuda",
                                         num_splits=c["splits"] if backend == "matched_splits" else 0)
        poison_workspace(res)
        plan = res.plan
        out = matched_decode(*g, resources=res, scale=scale).clone()
        lse = res.lse.clone()
        if backend == "matched_fused":
            fused = allocate_matched_resources(spec, "cuda", fused=True)
            poison_workspace(fused)
            single = matched_decode(*g, resources=fused, scale=scale)
            torch.cuda.synchronize()
            assert torch.equal(single.view(torch.int16), out.view(torch.int16)), where
        torch.cuda.synchronize()
        expected, _, lse_ref, bound, _, counts = OM.matched_decode_with_bounds(
            *case, plan.splits, plan.tokens_per_split, plan.tile_tokens, plan.lse_lanes, scale,
            counts=True)
        np.testing.assert_allclose(to_np(lse), lse_ref, atol=2e-5, rtol=1e-6, err_msg=where)
        assert_within_one_ulp(out, expected, where, bound, counts)
    else:
        res = allocate_resources(spec, "cuda", backend)
        if (index // len(BACKENDS)) % 2:
            res.chunk_maxima = res.chunk_denoms = res.chunk_accums = None   # the walk
        poison_workspace(res)
        out = paged_decode(*g, resources=res, backend=backend, scale=scale).clone()
        torch.cuda.synchronize()
        if backend == "hip_base":
            expected = OS.base_decode(*case, scale=scale)
        else:
            expected = OS.ml_merge(*OS.split_partitions(*case, spec.partitions, scale=scale))
        assert_within_one_ulp(out, expected, where)
    assert_close_dense(out, torch_dense(*g, scale=scale), where)
    for b, n in enumerate(c["lengths"]):
        if n == 0:
            assert torch.count_nonzero(out[b]) == 0, where


WALK_CASES = 16


def draw_walk(index):
    """A batch and an explicit split count whose (split, kv head, sequence) workgroups
    outnumber the CUs, in splits of 2 to 5 tiles: the partition walks several splits per
    workgroup."""
    from paged_decode.splitkv_plan import make_splitkv_plan
    rng = np.random.default_rng(9000 + index)
    dim = int(rng.choice([64, 128, 256]))
    hkv = int(rng.choice([4, 8]))
    group = int(rng.choice([1, 2, 4]))
    batch = int(rng.integers(8, 13))
    tile = 16384 // dim
    tiles = int(rng.integers(2, 6))
    splits = -(-257 // (hkv * batch)) + int(rng.integers(0, 3))
    capacity = max(tile, splits * tiles * tile - int(rng.integers(0, tile)))
    spec = DecodeSpec(batch, group * hkv, hkv, dim, capacity)
    # Page rounding of the capacity can add a tile per split: take the first split
    # count (from the drawn one up) whose splits hold 2 to 5 tiles.
    while True:
        plan = make_splitkv_plan(spec, 256, num_splits=splits)
        if 2 * tile <= plan.tokens_per_split <= 5 * tile:
            break
        splits += 1
    lengths = rng.integers(0, capacity + 1, size=batch)
    for b in range(batch):
        if rng.random() < 0.4:
            lengths[b] = min(int(rng.choice(BOUNDARIES + (capacity,))), capacity)
    scale = float(rng.uniform(0.02, 0.2)) if rng.random() < 0.25 else None
    return dict(dim=dim, hq=group * hkv, hkv=hkv, batch=batch, capacity=capacity,
                lengths=[int(x) for x in lengths], splits=splits, scale=scale, seed=index)


@pytest.mark.parametrize("index", range(WALK_CASES))
def test_random_walk_case(index):
    """The matched walk (several splits per workgroup) on seeded batches: bit for bit the
    single-launch path's output (one workgroup per split), and within the oracle's gate."""
    c = draw_walk(index)
    where = f"walk case {index}: {c}"
    q, k, v, table, lens = make_case(c["lengths"], c["hq"], c["hkv"], c["dim"], seed=c["seed"],
                                     capacity=c["capacity"])
    poison_tails(k, v, table, lens)
    case = (q, k, v, table, lens)
    g = to_gpu(case)
    spec = DecodeSpec(c["batch"], c["hq"], c["hkv"], c["dim"], c["capacity"])
    res = allocate_matched_resources(spec, "cuda", num_splits=c["splits"])
    plan = res.plan
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    assert plan.splits * c["hkv"] * c["batch"] > cus, where
    assert 2 * plan.tile_tokens <= plan.tokens_per_split <= 5 * plan.tile_tokens, where
    poison_workspace(res)
    out = matched_decode(*g, resources=res, scale=c["scale"]).clone()
    fused = allocate_matched_resources(spec, "cuda", num_splits=c["splits"], fused=True)
    poison_workspace(fused)
    single = matched_decode(*g, resources=fused, scale=c["scale"])
    torch.cuda.synchronize()
    assert torch.equal(single.view(torch.int16), out.view(torch.int16)), where
    assert torch.equal(fused.lse.view(torch.int32), res.lse.view(torch.int32)), where
    expected, _, lse_ref, bound, _, counts = OM.matched_decode_with_bounds(
        *case, plan.splits, plan.tokens_per_split, plan.tile_tokens, plan.lse_lanes, c["scale"],
        counts=True)
    np.testing.assert_allclose(to_np(res.lse), lse_ref, atol=2e-5, rtol=1e-6, err_msg=where)
    assert_within_one_ulp(out, expected, where, bound, counts)
    assert_close_dense(out, torch_dense(*g, scale=c["scale"]), where)
