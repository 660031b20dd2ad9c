"""The benchmark workloads at their full sizes, on the GPU.

Bandwidth sweep: batch 64, Hq 32, Hkv 8, D 128, lengths U[1, 32768] from a seed, every
sequence's pages scattered over the workload's 200 GB pool: 190,734 pages of 512 KiB per
cache (100 GB each, so element offsets pass 2^37), or the largest pool that fits the
device's free memory.  Edge coverage: batch 128, a quarter of the sequences empty, the
rest U[1, 4096] with page and partition boundaries, D 64 MHA 16/16 and D 256 GQA 32/4.

The CPU oracle cannot walk every sequence of these batches in seconds, so the checks are
* oracle parity (the one-bf16-ulp gate) on a few sequences, copied to the host with
  their pages, under the plan the full batch runs with;
* the dense fp32 device reference on every sequence at the reference's 2e-2 gate;
* properties that hold exactly at any size: moving every live page to other physical
  pages (and the table with it) leaves the output bit-identical; zeroing the lengths of
  half the batch leaves the other half bit-identical and gives exact zeros; a graph
  replay with new lengths equals the eager call.  The unused pool holds NaN, so any read
  outside the live tokens would show.
"""
import numpy as np
import pytest
import torch

if not torch.cuda.is_available():
    pytest.skip("needs an MI355X GPU", allow_module_level=True)

from gpu_cases import (assert_close_dense, assert_within_one_ulp, host_rows, poison_workspace,
                       pooled_case, to_np, torch_dense)
from parity import record
from oracle import matched as OM
from oracle import splitk as OS
from paged_decode.matched_splitkv import allocate_matched_resources, matched_decode
from paged_decode.runtime import allocate_resources, paged_decode
from paged_decode.spec import DecodeSpec

pytestmark = pytest.mark.gpu

SWEEP = dict(batch=64, hq=32, hkv=8, dim=128, capacity=32768, pool_pages=190734)
PAGE_BYTES = 256 * 8 * 128 * 2


def _sweep_pool_pages():
    """The 200 GB pool (K and V), capped at 80% of the free device memory.  A device with
    250 GB free (an MI355X has 288 GB) must hold the whole pool; the size used goes into the
    run's parity summary (pool_pages)."""
    free, _ = torch.cuda.mem_get_info()
    pages = min(SWEEP["pool_pages"], int(0.8 * free) // (2 * PAGE_BYTES))
    if free >= 250e9:
        assert pages == SWEEP["pool_pages"], f"{free / 1e9:.0f} GB free, pool cut to {pages}"
    print(f"bandwidth-sweep pool: {pages} pages per cache ({2 * pages * PAGE_BYTES / 1e9:.1f} GB)")
    record("bandwidth-sweep pool", pool_pages=pages)
    return pages


@pytest.fixture(autouse=True)
def _release_pool():
    yield
    torch.cuda.empty_cache()


def _bits(t):
    return t.contiguous().view(torch.int16)


def _sweep_lengths():
    return np.random.default_rng(64).integers(1, 32769, size=SWEEP["batch"]).astype(np.int32)


def _edge_lengths(batch=128, maximum=4096):
    rng = np.random.default_rng(404)
    lengths = rng.integers(1, maximum + 1, size=batch)
    lengths[rng.permutation(batch)[: batch // 4]] = 0
    special = [255, 256, 257, 511, 512, 513, 1023, 1024, 1025, 2047, 2048, 2049, maximum]
    lengths[batch // 4: batch // 4 + len(special)] = special
    return lengths.astype(np.int32)


def _sample_rows(lengths):
    """Longest, shortest non-empty and median sequence."""
    order = np.argsort(lengths, kind="stable")
    live = order[lengths[order] > 0]
    return sorted({int(live[-1]), int(live[0]), int(live[len(live) // 2])})


def _relocated(k, v, table, lengths):
    """Copies every live page to a free physical page of the same pool; returns the new
    table (the old pages keep their contents)."""
    live = table[table >= 0].long()
    used = torch.zeros(k.shape[0], dtype=torch.bool, device=k.device)
    used[live] = True
    free = torch.nonzero(~used).squeeze(1)
    assert free.numel() >= live.numel()
    gen = torch.Generator(device=k.device).manual_seed(5)
    target = free[torch.randperm(free.numel(), device=k.device, generator=gen)[: live.numel()]]
    k[target] = k[live]
    v[target] = v[live]
    moved = table.clone()
    moved[table >= 0] = target.to(torch.int32)
    return moved


def _check_exact_properties(call, q, k, v, table, lens):
    """call(q, k, v, table, lens) -> output tensor (borrowed)."""
    first = call(q, k, v, table, lens).clone()
    moved = _relocated(k, v, table, lens)
    assert torch.equal(_bits(call(q, k, v, moved, lens)), _bits(first)), "page relocation"
    half = lens.clone()
    half[1::2] = 0
    out = call(q, k, v, table, half).clone()
    assert torch.equal(_bits(out[0::2]), _bits(first[0::2])), "batch independence"
    assert torch.count_nonzero(out[1::2]) == 0
    return first


def _check_graph_replay(call, reset, q, k, v, table, lens):
    """Graph replays with new lengths equal eager calls; ``reset`` NaN-poisons the output
    and workspaces (outside the capture) before every replay and eager call."""
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    live = lens.clone()
    with torch.cuda.stream(stream):
        for _ in range(2):
            call(q, k, v, table, lens)
    torch.cuda.current_stream().wait_stream(stream)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = call(q, k, v, table, lens)
    # New lengths stay within each row's live pages (tensor contents are trusted).
    for values in (live // 3, torch.clamp(live - 255, min=0), live):
        lens.copy_(values)
        reset()
        graph.replay()
        captured = out.clone()
        reset()
        eager = call(q, k, v, table, lens).clone()
        assert torch.equal(_bits(captured), _bits(eager)), "graph replay"
    lens.copy_(live)


def test_bandwidth_sweep_matched_full_size():
    lengths = _sweep_lengths()
    g = pooled_case(lengths, SWEEP["hq"], SWEEP["hkv"], SWEEP["dim"], SWEEP["capacity"],
                    _sweep_pool_pages(), seed=64)
    spec = DecodeSpec(SWEEP["batch"], SWEEP["hq"], SWEEP["hkv"], SWEEP["dim"], SWEEP["capacity"])
    res = allocate_matched_resources(spec, "cuda")
    assert res.plan.splits == 1 and res.plan.tokens_per_split == 32768
    poison_workspace(res)

    def call(*args):
        return matched_decode(*args, resources=res)

    out = _check_exact_properties(call, *g)
    assert torch.isfinite(out).all()
    assert_close_dense(out, torch_dense(*g))
    rows = _sample_rows(lengths)
    host = host_rows(*g, rows)
    plan = res.plan
    expected, _, lse, bound, _, counts = OM.matched_decode_with_bounds(
        *host, plan.splits, plan.tokens_per_split, plan.tile_tokens, plan.lse_lanes,
        counts=True)
    out = call(*g)
    assert_within_one_ulp(out[rows], expected, f"sweep rows {rows}", bound, counts)
    np.testing.assert_allclose(to_np(res.lse[rows]), lse, atol=2e-5, rtol=1e-6)
    _check_graph_replay(call, lambda: poison_workspace(res), *g)


@pytest.mark.parametrize("backend", ["hip_base", "hip_splitk"])
def test_bandwidth_sweep_paged_backends_full_size(backend):
    lengths = _sweep_lengths()
    g = pooled_case(lengths, SWEEP["hq"], SWEEP["hkv"], SWEEP["dim"], SWEEP["capacity"],
                    _sweep_pool_pages(), seed=65)
    spec = DecodeSpec(SWEEP["batch"], SWEEP["hq"], SWEEP["hkv"], SWEEP["dim"], SWEEP["capacity"])
    res = allocate_resources(spec, "cuda", backend)
    poison_workspace(res)

    def call(*args):
        return paged_decode(*args, resources=res, backend=backend)

    out = _check_exact_properties(call, *g)
    assert_close_dense(out, torch_dense(*g))
    rows = _sample_rows(lengths)[:2]          # the longest and the shortest sequence
    host = host_rows(*g, rows)
    if backend == "hip_base":
        expected = OS.base_decode(*host)
    else:
        expected = OS.ml_merge(*OS.split_partitions(*host, spec.partitions))
    assert_within_one_ulp(call(*g)[rows], expected, f"{backend} sweep rows {rows}")
    _check_graph_replay(call, lambda: poison_workspace(res), *g)


@pytest.mark.parametrize("dim,hq,hkv", [(64, 16, 16), (256, 32, 4)])
def test_edge_coverage_full_batch_all_backends(dim, hq, hkv):
    lengths = _edge_lengths()
    g = pooled_case(lengths, hq, hkv, dim, 4096, pool_pages=8192, seed=404)
    spec = DecodeSpec(128, hq, hkv, dim, 4096)
    dense = torch_dense(*g)
    rows = _sample_rows(lengths) + [int(np.argmax(lengths == 2049))]
    host = host_rows(*g, rows)
    empty = torch.from_numpy(lengths == 0).cuda()
    for splits in (0, 3, 6):
        res = allocate_matched_resources(spec, "cuda", num_splits=splits)
        poison_workspace(res)
        out = matched_decode(*g, resources=res)
        assert_close_dense(out, dense)
        assert torch.count_nonzero(out[empty]) == 0
        plan = res.plan
        expected, _, _, bound, _, counts = OM.matched_decode_with_bounds(
            *host, plan.splits, plan.tokens_per_split, plan.tile_tokens, plan.lse_lanes,
            counts=True)
        assert_within_one_ulp(out[rows], expected, f"matched {plan.splits} splits", bound,
                              counts)
    for backend in ("hip_base", "hip_splitk"):
        res = allocate_resources(spec, "cuda", backend)
        poison_workspace(res)
        out = paged_decode(*g, resources=res, backend=backend)
        assert_close_dense(out, dense)
        assert torch.count_nonzero(out[empty]) == 0
        if backend == "hip_base":
            expected = OS.base_decode(*host)
        else:
            expected = OS.ml_merge(*OS.split_partitions(*host, spec.partitions))
        assert_within_one_ulp(out[rows], expected, backend)
