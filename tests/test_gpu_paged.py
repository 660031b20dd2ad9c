"""GPU parity of paged_decode backends hip_base and hip_splitk (and their aliases).

Restates the reference's tests/test_gpu.py:51-128 and adds oracle parity at one
bf16 ulp against oracle/splitk.py (the reference kernels.py restated).

Most cases run twice, once per grid of paged_decode: the walk (one workgroup per
kv head group and sequence, resources without the chunk workspace) and the
small-batch chunks (the table width cut into partitions of one workgroup each,
then merged), which every batch of fewer walks than half the CUs takes.  Every
output and workspace is NaN-poisoned before a call, as the reference does
(tools/resident_experiment.py:117-121).
"""
import numpy as np
import pytest
import torch

if not torch.cuda.is_available():
    pytest.skip("needs an MI355X GPU", allow_module_level=True)

from cases import make_case, poison_tails
from gpu_cases import (assert_close_dense, assert_within_one_ulp, poison, poison_workspace,
                       to_gpu, to_np, torch_dense)
from oracle import splitk as OS
from paged_decode import _native
from paged_decode.runtime import (_chunk_plan, allocate_resources, paged_decode,
                                  validate_device_metadata)
from paged_decode.spec import DecodeSpec, canonical_backend

pytestmark = pytest.mark.gpu

BACKENDS = ["hip_base", "hip_splitk", "triton_base", "triton_splitk"]
GRIDS = ["walk", "chunks"]


def resources_for(spec, backend, grid):
    """Resources whose calls take ``grid``: "walk" drops the chunk workspace (so every
    batch takes the walk), "chunks" keeps it.  Output and workspaces are NaN."""
    res = allocate_resources(spec, "cuda", backend)
    if grid == "walk":
        res.chunk_maxima = res.chunk_denoms = res.chunk_accums = None
    poison_workspace(res)
    return res


def assert_grid(res, g, grid):
    """The call of case ``g`` on ``res`` takes ``grid``."""
    chunked = _chunk_plan(res, g[0].shape[0], g[3].shape[1]) is not None
    assert chunked == (grid == "chunks"), f"expected the {grid} grid"


def oracle_for(case, backend, spec, scale=None):
    if canonical_backend(backend) == "hip_base":
        return OS.base_decode(*case, scale=scale)
    return OS.ml_merge(*OS.split_partitions(*case, spec.partitions, scale=scale))


@pytest.mark.parametrize("grid", GRIDS)
@pytest.mark.parametrize("backend", BACKENDS)
@pytest.mark.parametrize("dim,hq,hkv", [(64, 4, 1), (128, 4, 2), (64, 2, 2), (256, 8, 2)])
def test_boundaries_gqa_and_padding(backend, dim, hq, hkv, grid):
    lengths = [0, 1, 255, 256, 257, 1023, 1024, 1025]
    q, k, v, table, lens = make_case(lengths, hq, hkv, dim, seed=19, capacity=1025)
    poison_tails(k, v, table, lens)
    case = (q, k, v, table, lens)
    g = to_gpu(case)
    validate_device_metadata(g[3], g[4], len(k), 1025)
    spec = DecodeSpec(len(lengths), hq, hkv, dim, 1025)
    res = resources_for(spec, backend, grid)
    assert_grid(res, g, grid)
    actual = paged_decode(*g, resources=res, backend=backend).clone()
    torch.cuda.synchronize()
    assert_close_dense(actual, torch_dense(*g))
    assert_within_one_ulp(actual, oracle_for(case, backend, spec), f"{backend} {grid}")
    assert torch.count_nonzero(actual[0]) == 0


@pytest.mark.parametrize("grid", GRIDS)
@pytest.mark.parametrize("backend", ["hip_base", "hip_splitk"])
@pytest.mark.parametrize("dim,hq,hkv", [(64, 4, 1), (256, 4, 1), (64, 8, 2)])
def test_graph_replay_changes_lengths_pages_and_kv(backend, dim, hq, hkv, grid):
    case = make_case([255, 1023, 0], hq, hkv, dim, seed=19, capacity=2048)
    g = to_gpu(case)
    q, k, v, table, lens = g
    spec = DecodeSpec(3, hq, hkv, dim, 2048)
    res = resources_for(spec, backend, grid)
    assert_grid(res, g, grid)
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        for _ in range(3):
            paged_decode(*g, resources=res, backend=backend)
    torch.cuda.current_stream().wait_stream(stream)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        output = paged_decode(*g, resources=res, backend=backend)
    for lengths in ([256, 1024, 0], [257, 1025, 1], [1, 0, 1025], [0, 0, 0], [2048, 2047, 1]):
        lens.copy_(torch.tensor(lengths, device="cuda", dtype=torch.int32))
        q.normal_()
        k.normal_()
        v.normal_()
        table.copy_(table.flip(1))
        poison_workspace(res)
        graph.replay()
        captured = output.clone()
        torch.cuda.synchronize()
        host = (to_np(q), to_np(k), to_np(v), table.cpu().numpy(), lens.cpu().numpy())
        assert_close_dense(captured, torch_dense(*g))
        assert_within_one_ulp(captured, oracle_for(host, backend, spec),
                              f"{grid} replay {lengths}")
        poison_workspace(res)
        eager = paged_decode(*g, resources=res, backend=backend).clone()
        torch.testing.assert_close(captured, eager, atol=0, rtol=0)


def test_public_contract_rejects_bad_dtype_and_missing_workspace():
    g = to_gpu(make_case([2], 4, 1, 64, capacity=2048))
    r = allocate_resources(DecodeSpec(1, 4, 1, 64, 2048), "cuda", "hip_base")
    for backend in ("hip_splitk", "triton_splitk"):
        with pytest.raises(ValueError, match="workspace"):
            paged_decode(*g, resources=r, backend=backend)
    with pytest.raises(ValueError, match="BF16"):
        paged_decode(g[0].float(), *g[1:], resources=r)
    with pytest.raises(ValueError, match="unknown decode_backend"):
        paged_decode(*g, resources=r, backend="triton_tc")
    with pytest.raises(ValueError, match="resources require a custom backend"):
        allocate_resources(DecodeSpec(1, 4, 1, 64, 2048), "cuda", "flash_attn")


@pytest.mark.parametrize("grid", GRIDS)
@pytest.mark.parametrize("backend", ["hip_splitk"])
@pytest.mark.parametrize("dim", [64, 256])
def test_non_power_of_two_split_count(dim, backend, grid):
    # Three real partitions (reference tests/test_gpu.py:121-128).
    case = make_case([0, 2051, 2049, 1025], 4, 1, dim, seed=19, capacity=2051)
    g = to_gpu(case)
    spec = DecodeSpec(4, 4, 1, dim, 2051)
    res = resources_for(spec, backend, grid)
    assert_grid(res, g, grid)
    actual = paged_decode(*g, resources=res, backend=backend)
    torch.cuda.synchronize()
    assert_close_dense(actual, torch_dense(*g))
    assert_within_one_ulp(actual, oracle_for(case, backend, spec))


@pytest.mark.parametrize("grid", GRIDS)
@pytest.mark.parametrize("backend", ["hip_base", "hip_splitk"])
def test_eager_partial_batch_and_live_table_width(backend, grid):
    # The scheduler may pass fewer rows than max_batch and only the live width.
    case = make_case([300, 5, 511], 8, 2, 128, seed=7, capacity=512)
    g = to_gpu(case)
    spec = DecodeSpec(6, 8, 2, 128, 4096)
    res = resources_for(spec, backend, grid)
    assert_grid(res, g, grid)
    actual = paged_decode(*g, resources=res, backend=backend, scale=0.1)
    torch.cuda.synchronize()
    assert actual.shape == (3, 8, 128)
    # Rows past the live batch are never written: they keep the NaN poison.
    assert torch.isnan(res.out[3:].float()).all()
    assert_close_dense(actual, torch_dense(*g, scale=0.1))
    assert_within_one_ulp(actual, oracle_for(case, backend, spec, scale=0.1))


@pytest.mark.parametrize("grid", GRIDS)
@pytest.mark.parametrize("backend", ["hip_base", "hip_splitk"])
@pytest.mark.parametrize("dim,hq,hkv", [(64, 16, 16), (256, 32, 4)])
def test_edge_coverage_config_c4(backend, dim, hq, hkv, grid):
    rng = np.random.default_rng(404)
    lengths = rng.integers(1, 4097, size=32)
    lengths[:8] = 0
    lengths[8:20] = [255, 256, 257, 511, 512, 513, 1023, 1024, 1025, 2047, 2048, 4096]
    case = make_case(list(lengths.astype(np.int32)), hq, hkv, dim, seed=5, capacity=4096)
    g = to_gpu(case)
    spec = DecodeSpec(32, hq, hkv, dim, 4096)
    res = resources_for(spec, backend, grid)
    assert_grid(res, g, grid)
    actual = paged_decode(*g, resources=res, backend=backend)
    torch.cuda.synchronize()
    assert_close_dense(actual, torch_dense(*g))
    assert_within_one_ulp(actual, oracle_for(case, backend, spec))
    assert torch.count_nonzero(actual[:8]) == 0


@pytest.mark.parametrize("grid", GRIDS)
@pytest.mark.parametrize("backend", ["hip_base", "hip_splitk"])
def test_context_beyond_the_prefetched_table_window(backend, grid):
    # The walk reads 80 pages in one workgroup, past its 128-entry table window's
    # first half; the chunks start their windows at their own first pages.
    case = make_case([20480, 17000, 3], 4, 1, 128, seed=9, capacity=20480)
    g = to_gpu(case)
    spec = DecodeSpec(3, 4, 1, 128, 20480)
    res = resources_for(spec, backend, grid)
    assert_grid(res, g, grid)
    actual = paged_decode(*g, resources=res, backend=backend)
    torch.cuda.synchronize()
    assert_close_dense(actual, torch_dense(*g))
    assert_within_one_ulp(actual, oracle_for(case, backend, spec))



@pytest.mark.parametrize("grid", GRIDS)
@pytest.mark.parametrize("backend", ["hip_base", "hip_splitk"])
@pytest.mark.parametrize("dim,hq,hkv", [(128, 32, 1), (64, 24, 1), (256, 40, 2), (128, 17, 1)])
def test_groups_larger_than_16_heads(backend, dim, hq, hkv, grid):
    """A kv head with more than 16 query heads is served in 16-head slices (the reference
    grid has no group limit for these backends)."""
    lengths = [0, 1, 300, 1100]
    q, k, v, table, lens = make_case(lengths, hq, hkv, dim, seed=23, capacity=1100)
    poison_tails(k, v, table, lens)
    case = (q, k, v, table, lens)
    g = to_gpu(case)
    spec = DecodeSpec(len(lengths), hq, hkv, dim, 1100)
    res = resources_for(spec, backend, grid)
    assert_grid(res, g, grid)
    actual = paged_decode(*g, resources=res, backend=backend).clone()
    torch.cuda.synchronize()
    assert_close_dense(actual, torch_dense(*g))
    assert_within_one_ulp(actual, oracle_for(case, backend, spec),
                          f"{backend} {grid} G={hq // hkv}")
    assert torch.count_nonzero(actual[0]) == 0


@pytest.mark.parametrize("grid", GRIDS)
@pytest.mark.parametrize("backend", ["hip_base", "hip_splitk"])
def test_d256_tile_counts_of_the_loader_kernel(backend, grid):
    """D=256 runs cols_loader_kernel for both backends: whole contexts (base) and
    1024-token partitions (split) of 1 to 20 tiles, full and partial: the loader
    wavefronts' prologue and waits differ for one, two and more tiles."""
    lengths = [1, 64, 65, 129, 192, 255, 320, 1023, 1024, 1025, 1100, 1280]
    q, k, v, table, lens = make_case(lengths, 8, 2, 256, seed=43, capacity=1280)
    poison_tails(k, v, table, lens)
    case = (q, k, v, table, lens)
    g = to_gpu(case)
    spec = DecodeSpec(len(lengths), 8, 2, 256, 1280)
    res = resources_for(spec, backend, grid)
    assert_grid(res, g, grid)
    actual = paged_decode(*g, resources=res, backend=backend).clone()
    torch.cuda.synchronize()
    assert_close_dense(actual, torch_dense(*g))
    assert_within_one_ulp(actual, oracle_for(case, backend, spec), f"{backend} {grid}")


def split_fixed_rows(g, hkv, parts, part, rows=None, decode=False):
    """pd_split_fixed over case ``g`` with its batch padded by empty sequences (-1 tables,
    zero queries) to ``rows`` rows (None: as it is); the (m, l, acc) of the case's own rows.
    With ``decode``, pd_split_decode instead, and its merged output as a fourth value.
    The workspaces and the output start NaN."""
    q, k, v, table, lens = g
    b = q.shape[0]
    if rows is not None and rows > b:
        q = torch.cat([q, torch.zeros((rows - b, *q.shape[1:]), device="cuda", dtype=q.dtype)])
        table = torch.cat([table, torch.full((rows - b, table.shape[1]), -1, device="cuda",
                                             dtype=table.dtype)])
        lens = torch.cat([lens, torch.zeros(rows - b, device="cuda", dtype=lens.dtype)])
    n, hq, dim = q.shape
    maxima = torch.full((n, hq, parts), float("nan"), device="cuda")
    denoms = torch.full_like(maxima, float("nan"))
    accums = torch.full((n, hq, parts, dim), float("nan"), device="cuda")
    if not decode:
        _native.split_fixed(q, k, v, table, lens, maxima, denoms, accums, hkv, parts, part,
                            dim ** -0.5)
        return maxima[:b], denoms[:b], accums[:b]
    out = torch.full((n, hq, dim), float("nan"), device="cuda", dtype=torch.bfloat16)
    _native.split_decode(q, k, v, table, lens, maxima, denoms, accums, out, hkv, parts, part,
                         dim ** -0.5)
    return maxima[:b], denoms[:b], accums[:b], out[:b]


@pytest.mark.parametrize("dim,hq,hkv", [(64, 4, 1), (128, 8, 2), (256, 8, 2), (64, 32, 2),
                                         (64, 8, 2), (64, 6, 6), (64, 16, 16), (64, 12, 4),
                                         (256, 40, 2)])
@pytest.mark.parametrize("tiles_per_partition", [1, 2, 3, 5])
def test_fixed_split_grids_and_partition_sizes(dim, hq, hkv, tiles_per_partition):
    """pd_split_fixed runs one workgroup per partition when its walks (one workgroup per kv
    head group and sequence) are fewer than the CUs, as here, and one walking workgroup per
    (kv head group, sequence), writing every partition as it leaves it, when the walks fill
    the CUs (the same sequences followed by empty ones).  Both grids must write the same
    (m, l, acc) bits.  pd_split_decode on either grid (one workgroup per partition, then its
    online merge; or the walk, whose workgroups merge their own partitions) must write the
    same workspace and the same output bits, within one ulp of the oracle.  Partition
    sizes of 1, 2, 3 and 5 tiles, lengths at and around partition and page boundaries,
    the empty partitions past each sequence's end, and NaN-poisoned tails: the workspace
    against oracle/splitk.py, and the merged output at one bf16 ulp."""
    tile = 16384 // dim
    part = tiles_per_partition * tile
    cap = 4 * part + 3 * tile
    lengths = [0, 1, tile, part - 1, part, part + 1, 2 * part + tile // 2, cap]
    check_fixed_split_grids(dim, hq, hkv, part, lengths, cap, tiles_per_partition,
                            f"D{dim} {hq}/{hkv} {tiles_per_partition}-tile partitions")


@pytest.mark.parametrize("dim,hq,hkv", [(64, 2, 1), (64, 4, 1), (128, 8, 2), (128, 8, 1),
                                         (128, 16, 1), (256, 8, 1), (256, 16, 1), (256, 40, 2)])
def test_fixed_split_walk_of_more_partitions_than_a_hold(dim, hq, hkv):
    """The walk holds up to 16, 8 or 4 completed partitions in the loaders' registers (by
    the one, two or four 16-byte stores each loader lane makes per partition) and stores a
    full hold before taking the next one; with one-tile partitions and up to 37 of them
    per sequence, the holds fill and are stored two to nine times in one walk.  The same
    checks as above."""
    tile = 16384 // dim
    cap = 37 * tile
    lengths = [cap, cap - 1, 16 * tile + 1, 8 * tile, 4 * tile + 3, 1, 0, 33 * tile]
    check_fixed_split_grids(dim, hq, hkv, tile, lengths, cap, 37,
                            f"D{dim} {hq}/{hkv} 37 one-tile partitions")


def check_fixed_split_grids(dim, hq, hkv, part, lengths, cap, seed, label):
    q, k, v, table, lens = make_case(lengths, hq, hkv, dim, seed=seed, capacity=cap)
    poison_tails(k, v, table, lens)
    case = (q, k, v, table, lens)
    g = to_gpu(case)
    parts = -(-cap // part)
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    maxima, denoms, accums = split_fixed_rows(g, hkv, parts, part)
    walked = split_fixed_rows(g, hkv, parts, part, rows=cus)
    for one, other in zip((maxima, denoms, accums), walked):
        assert torch.equal(one.view(torch.int32), other.view(torch.int32))
    out = torch.full((len(lengths), hq, dim), float("nan"), device="cuda", dtype=torch.bfloat16)
    _native.ml_merge(maxima, denoms, accums, out, len(lengths))
    decoded = []
    for rows in (None, cus):
        *workspace, merged = split_fixed_rows(g, hkv, parts, part, rows=rows, decode=True)
        for one, other in zip((maxima, denoms, accums), workspace):
            assert torch.equal(one.view(torch.int32), other.view(torch.int32)), rows
        decoded.append(merged)
    assert torch.equal(decoded[0].view(torch.int16), decoded[1].view(torch.int16)), \
        "pd_split_decode: the walk and one workgroup per partition differ"
    torch.cuda.synchronize()
    m_ref, l_ref, a_ref = OS.split_partitions(*case, parts, part_size=part)
    assert_within_one_ulp(decoded[0], OS.ml_merge(m_ref, l_ref, a_ref), f"pd_split_decode {label}")
    np.testing.assert_array_equal(np.isinf(to_np(maxima)), np.isinf(m_ref))
    live = np.isfinite(m_ref)
    np.testing.assert_allclose(to_np(maxima)[live], m_ref[live], rtol=1e-6, atol=1e-6)
    np.testing.assert_allclose(to_np(denoms), l_ref, rtol=3e-5, atol=1e-6)
    np.testing.assert_allclose(to_np(accums), a_ref, rtol=3e-5, atol=3e-5)
    assert_within_one_ulp(out, OS.ml_merge(m_ref, l_ref, a_ref), label)
    assert torch.count_nonzero(out[lengths.index(0)]) == 0


@pytest.mark.parametrize("grid", GRIDS)
@pytest.mark.parametrize("backend", ["hip_base", "hip_splitk"])
@pytest.mark.parametrize("hq,hkv", [(2, 2), (16, 16), (8, 4), (6, 2), (16, 2), (12, 4), (10, 2),
                                    (4, 4), (16, 4), (3, 3)])
def test_d64_kv_head_groups(backend, hq, hkv, grid):
    """At D=64 one workgroup serves four adjacent kv heads and their 4G query heads when
    the kv head count is a multiple of 4 and 4G <= 16 (tiles of 64 tokens of the four
    heads), else two when it is even and 2G <= 16 (128-token tiles); odd kv head counts
    stay one per workgroup.  Group sizes 1 to 8 (padded to 2, 4, 8 and 16 query heads),
    lengths around the 64- and 128-token tile boundaries and the partitions,
    NaN-poisoned tails."""
    lengths = [0, 1, 2, 63, 64, 65, 127, 128, 129, 255, 256, 257, 383, 511, 512, 513, 1100]
    q, k, v, table, lens = make_case(lengths, hq, hkv, 64, seed=hq * 31 + hkv, capacity=1100)
    poison_tails(k, v, table, lens)
    case = (q, k, v, table, lens)
    g = to_gpu(case)
    spec = DecodeSpec(len(lengths), hq, hkv, 64, 1100)
    res = resources_for(spec, backend, grid)
    assert_grid(res, g, grid)
    actual = paged_decode(*g, resources=res, backend=backend).clone()
    torch.cuda.synchronize()
    assert_close_dense(actual, torch_dense(*g), f"{backend} {grid} {hq}/{hkv}")
    assert_within_one_ulp(actual, oracle_for(case, backend, spec), f"{backend} {grid} {hq}/{hkv}")
    assert torch.count_nonzero(actual[0]) == 0


@pytest.mark.parametrize("backend", ["hip_base", "hip_splitk"])
@pytest.mark.parametrize("batch", [1, 8])
@pytest.mark.parametrize("hq,hkv,dim,cap,ctx", [(16, 4, 256, 2112, 2064),
                                                 (32, 8, 128, 4096, 4096)])
def test_small_batch_chunks_on_benchmark_shapes(backend, batch, hq, hkv, dim, cap, ctx):
    """The small-batch shapes of the benchmark (D256 GQA 16/4 at context 2064, D128 GQA 32/8
    at 4096; B = 1 and 8) take the chunks: the table width cut into ~256 / (B x kv heads)
    partitions of one workgroup each, merged by pd_ml_merge.  The output passes the
    backend's oracle gate (base: one online softmax over the context; splitk: 1024-token
    partitions merged) and the dense gate, like the walk's, from NaN-poisoned workspaces."""
    rng = np.random.default_rng(batch * 7 + dim)
    lengths = [ctx] + [int(x) for x in rng.integers(0, ctx + 1, size=batch - 1)]
    q, k, v, table, lens = make_case(lengths, hq, hkv, dim, seed=batch + dim, capacity=cap)
    poison_tails(k, v, table, lens)
    case = (q, k, v, table, lens)
    g = to_gpu(case)
    spec = DecodeSpec(batch, hq, hkv, dim, cap)
    expected = oracle_for(case, backend, spec)
    dense = torch_dense(*g)
    outputs = {}
    for grid in GRIDS:
        res = resources_for(spec, backend, grid)
        assert_grid(res, g, grid)
        outputs[grid] = paged_decode(*g, resources=res, backend=backend).clone()
        torch.cuda.synchronize()
        where = f"{backend} {grid} B={batch} D{dim} {hq}/{hkv} ctx {ctx}"
        assert_close_dense(outputs[grid], dense, where)
        assert_within_one_ulp(outputs[grid], expected, where)
    chunks, tokens = _chunk_plan(res, batch, g[3].shape[1])
    print(f"B={batch} D{dim} {hq}/{hkv}: {chunks} chunks of {tokens} tokens")


@pytest.mark.parametrize("backend", ["hip_base", "hip_splitk"])
@pytest.mark.parametrize("hq,hkv,dim", [(16, 4, 256), (16, 16, 64), (8, 2, 128)])
def test_chunks_do_not_depend_on_padding_or_the_live_width(backend, hq, hkv, dim):
    """The small-batch chunks give a sequence the same bits whether it runs in the live
    batch with the live table width (an eager engine step) or in a batch padded with empty
    sequences up to its next power of two over capacity-wide tables (the step's decode
    graph bucket), which run more, trailing empty, chunks."""
    lengths = [1000, 700, 1]
    case = make_case(lengths, hq, hkv, dim, seed=hq + dim, capacity=1000)
    poison_tails(*case[1:])
    g = to_gpu(case)
    q, k, v, table, lens = g
    spec = DecodeSpec(8, hq, hkv, dim, 2112)
    res = resources_for(spec, backend, "chunks")
    live = paged_decode(*g, resources=res, backend=backend).clone()
    bucket, width = 4, spec.table_width
    qp = torch.zeros((bucket, hq, dim), device="cuda", dtype=q.dtype)
    qp[:3] = q
    tp = torch.full((bucket, width), -1, device="cuda", dtype=torch.int32)
    tp[:3, :table.shape[1]] = table
    lp = torch.zeros(bucket, device="cuda", dtype=torch.int32)
    lp[:3] = lens
    assert _chunk_plan(res, 3, table.shape[1])[0] < _chunk_plan(res, bucket, width)[0]
    poison_workspace(res)
    padded = paged_decode(qp, k, v, tp, lp, resources=res, backend=backend).clone()
    torch.cuda.synchronize()
    assert torch.equal(padded[:3].view(torch.int16), live.view(torch.int16))
    assert torch.count_nonzero(padded[3]) == 0
    assert_within_one_ulp(live, oracle_for(case, backend, spec), f"{backend} D{dim} {hq}/{hkv}")


@pytest.mark.parametrize("dim", [64, 128, 256])
@pytest.mark.parametrize("parts", [1, 3, 4, 5, 9, 16, 17, 33, 48, 49, 100, 128, 129, 200])
def test_ml_merge_rows_partitions_and_alignment(dim, parts):
    """pd_ml_merge over seeded (m, l, acc) states with empty partitions (m = -inf, l = 0,
    acc = 0) and an all-empty row, against the oracle's merge at one bf16 ulp.  Up to 128
    partitions the kernel takes one wavefront per row (rows >= 2048, 16-byte aligned
    accumulators) or per 64 columns, and loads in batches sized to the partition count:
    the same rows give the same bits alone, among 2048 rows, and from unaligned
    accumulators."""
    rng = np.random.default_rng(parts * 3 + dim)
    b, hq = 2, 4
    m = (rng.normal(size=(b, hq, parts)) * 3).astype(np.float32)
    l = rng.uniform(0.5, 40, size=(b, hq, parts)).astype(np.float32)
    acc = (rng.normal(size=(b, hq, parts, dim)) * l[..., None]).astype(np.float32)
    empty = rng.random((b, hq, parts)) < 0.3
    empty[1, 2] = True                                    # an all-empty row
    m[empty], l[empty], acc[empty] = -np.inf, 0, 0
    expected = OS.ml_merge(m, l, acc)

    def merge(mm, ll, aa, rows_b):
        out = torch.full((rows_b, hq, dim), float("nan"), device="cuda", dtype=torch.bfloat16)
        _native.ml_merge(mm, ll, aa, out, rows_b)
        return out

    gm, gl, ga = (torch.from_numpy(x).cuda() for x in (m, l, acc))
    alone = merge(gm, gl, ga, b)
    reps = 2048 // (b * hq)
    many = merge(gm.repeat(reps, 1, 1), gl.repeat(reps, 1, 1), ga.repeat(reps, 1, 1, 1), b * reps)
    storage = torch.empty(ga.numel() + 1, device="cuda")
    unaligned = storage[1:].view(ga.shape)
    unaligned.copy_(ga)
    odd = merge(gm, gl, unaligned, b)
    torch.cuda.synchronize()
    assert_within_one_ulp(alone, expected, f"ml_merge D{dim} {parts} partitions")
    assert torch.count_nonzero(alone[1, 2]) == 0
    for other in (many[:b], many[-b:], odd):
        assert torch.equal(other.view(torch.int16), alone.view(torch.int16))
