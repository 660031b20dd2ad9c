"""GPU parity of the matched split-KV operator (pd_partition + pd_lse_merge).

Outputs are compared with the CPU oracle (oracle/matched.py) at one bf16 ulp
and with the dense fp32 reference at the reference's 2e-2 gate.  Cases follow
the reference's tests/test_matched_splitkv.py and the benchmark geometries.
"""
import numpy as np
import pytest
import torch

if not torch.cuda.is_available():
    pytest.skip("needs an MI355X GPU", allow_module_level=True)

from cases import make_case, poison_tails
from gpu_cases import (assert_close_dense, assert_within_one_ulp, poison, poison_workspace,
                       to_gpu, to_np, torch_dense)
from oracle import matched as OM
from paged_decode import _native
from paged_decode.matched_splitkv import allocate_matched_resources, matched_decode
from paged_decode.spec import DecodeSpec

pytestmark = pytest.mark.gpu


def oracle_for(case, plan, scale=None):
    """(out, partials, lse, rounding-ambiguity bound of out) from the oracle."""
    return OM.matched_decode_with_bounds(*case, plan.splits, plan.tokens_per_split,
                                         plan.tile_tokens, plan.lse_lanes, scale, counts=True)


def run(case, spec, num_splits=0, scale=None):
    g = to_gpu(case)
    res = allocate_matched_resources(spec, "cuda", num_splits=num_splits)
    poison_workspace(res)
    out = matched_decode(*g, resources=res, scale=scale)
    torch.cuda.synchronize()
    return g, res, out


def assert_partials(actual, expected, bound):
    """fp32 partials: within the oracle's rounding-ambiguity bound plus fp32 noise."""
    diff = np.abs(to_np(actual) - expected)
    allowed = bound + 2e-5 + 2e-5 * np.abs(expected)
    assert (diff <= allowed).all(), f"partials off by up to {diff.max():.3g}"


def check_all(case, g, res, out, scale=None, where=""):
    expected, partials, lse, bound, partial_bound, counts = oracle_for(case, res.plan, scale)
    frac = assert_within_one_ulp(out, expected, where, bound, counts)
    np.testing.assert_allclose(to_np(res.lse), lse, atol=2e-5, rtol=1e-6)
    assert_partials(res.partials, partials, partial_bound)
    assert_close_dense(out, torch_dense(*g, scale=scale))
    return frac


@pytest.mark.parametrize("ctx,cap", [(528, 528), (2064, 2112), (2064, 2064), (2112, 2112),
                                     (1, 2112), (2063, 2304)])
def test_d256_gqa_single_sequence(ctx, cap):
    case = make_case([ctx], 16, 4, 256, seed=20261105, capacity=cap)
    g, res, out = run(case, DecodeSpec(1, 16, 4, 256, cap))
    frac = check_all(case, g, res, out, where=f"ctx {ctx}")
    print(f"plan {res.plan.splits}x{res.plan.tokens_per_split} sm {res.plan.sm_count}: "
          f"{frac:.2e} of outputs one ulp off")


@pytest.mark.parametrize("lengths,hq,hkv,dim,cap", [
    ([2064, 0, 1000, 1, 64, 65], 16, 4, 256, 2112),
    ([4096, 0, 300, 2049], 32, 8, 128, 4096),
    ([1000, 0, 1, 257, 256], 16, 16, 64, 1024),
    ([700, 0, 33], 8, 1, 128, 768),
])
def test_one_split_plan_writes_its_output_in_the_partition(lengths, hq, hkv, dim, cap):
    """A plan of one split of several tiles needs no merge launch: the LSE merge weighs
    that split by exactly 1, so matched_decode (pd_matched_decode without counters) lets
    the partition write bf16(partial) itself.  Output, partials and LSEs must equal
    pd_partition + pd_lse_merge's bit for bit (NaN-poisoned buffers; zero-length rows
    exactly 0), and the output the oracle's at one ulp."""
    case = make_case(lengths, hq, hkv, dim, seed=len(lengths) + dim, capacity=cap)
    poison_tails(*case[1:])
    spec = DecodeSpec(len(lengths), hq, hkv, dim, cap)
    g, res, out = run(case, spec, num_splits=1)
    plan = res.plan
    assert plan.splits == 1 and plan.tokens_per_split > plan.tile_tokens
    partials = torch.full_like(res.partials, float("nan"))
    lse = torch.full_like(res.lse, float("nan"))
    two = torch.full_like(out, float("nan"))
    _native.partition(*g, partials, lse, hkv, 1, plan.tokens_per_split, plan.tile_tokens,
                      dim ** -0.5)
    _native.lse_merge(partials, lse, two, plan.lse_lanes)
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), two.view(torch.int16)), \
        "one-split output differs from pd_partition + pd_lse_merge"
    assert torch.equal(res.partials.view(torch.int32), partials.view(torch.int32))
    assert torch.equal(res.lse.view(torch.int32), lse.view(torch.int32))
    for i, n in enumerate(lengths):
        if n == 0:
            assert torch.count_nonzero(out[i].view(torch.int16)) == 0
    check_all(case, g, res, out, where=f"one split D{dim} {hq}/{hkv}")


def test_d256_fixed_1024_token_partitions():
    """Same kernels with 1024-token partitions (the fixed-partition geometry)."""
    case = make_case([2064], 16, 4, 256, seed=20261105, capacity=2112)
    g = to_gpu(case)
    partials = torch.full((1, 16, 3, 256), float("nan"), device="cuda", dtype=torch.float32)
    lse = torch.full((1, 16, 3), float("nan"), device="cuda", dtype=torch.float32)
    out = torch.full((1, 16, 256), float("nan"), device="cuda", dtype=torch.bfloat16)
    _native.partition(*g, partials, lse, 4, 3, 1024, 64, 256 ** -0.5)
    _native.lse_merge(partials, lse, out, 4)
    torch.cuda.synchronize()
    expected, _, exp_lse, bound, _, counts = OM.matched_decode_with_bounds(*case, 3, 1024, 64,
                                                                           4, counts=True)
    assert_within_one_ulp(out, expected, "1024-token partitions", bound, counts)
    np.testing.assert_allclose(to_np(lse), exp_lse, atol=2e-5, rtol=1e-6)


@pytest.mark.parametrize("splits", [3, 6])
@pytest.mark.parametrize("dim,hq,hkv", [(64, 4, 1), (128, 4, 2), (256, 8, 2)])
def test_explicit_cross_page_boundaries(splits, dim, hq, hkv):
    # reference tests/test_matched_splitkv.py:20-36, with NaN tails and -1 padding.
    lengths = [0, 1, 255, 256, 257, 1023, 1024, 2051]
    q, k, v, table, lens = make_case(lengths, hq, hkv, dim, capacity=2051)
    poison_tails(k, v, table, lens)
    case = (q, k, v, table, lens)
    g, res, out = run(case, DecodeSpec(8, hq, hkv, dim, 2051), num_splits=splits)
    check_all(case, g, res, out)
    assert torch.count_nonzero(out[0]) == 0


def test_graph_replay_and_empty_partitions():
    # reference tests/test_matched_splitkv.py:39-57: capture after warmup, then
    # replay with new lengths, pages and KV; replay == eager bit-exactly.
    case = make_case([255, 1023, 0], 8, 2, 256, capacity=2051)
    q, k, v, table, lengths = g = to_gpu(case)
    res = allocate_matched_resources(DecodeSpec(3, 8, 2, 256, 2051), "cuda")
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        for _ in range(3):
            matched_decode(*g, resources=res)
    torch.cuda.current_stream().wait_stream(stream)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = matched_decode(*g, resources=res)
    for values in ([257, 1025, 0], [2051, 1, 0], [0, 0, 0], [2051, 2051, 2051]):
        lengths.copy_(torch.tensor(values, dtype=torch.int32, device="cuda"))
        q.normal_()
        k.normal_()
        v.normal_()
        table.copy_(table.flip(1))
        poison_workspace(res)
        graph.replay()
        captured = out.clone()
        torch.cuda.synchronize()
        host = (to_np(q), to_np(k), to_np(v), table.cpu().numpy(), lengths.cpu().numpy())
        expected, _, _, bound, _, counts = oracle_for(host, res.plan)
        assert_within_one_ulp(captured, expected, f"replay {values}", bound, counts)
        assert_close_dense(captured, torch_dense(*g))
        poison_workspace(res)
        eager = matched_decode(*g, resources=res)
        torch.testing.assert_close(captured, eager, atol=0, rtol=0)
        if not any(values):
            assert torch.count_nonzero(captured) == 0


def _two_kernel_resources(res):
    from paged_decode.matched_splitkv import MatchedResources
    return MatchedResources(res.spec, res.plan, torch.empty_like(res.out),
                            torch.empty_like(res.partials), torch.empty_like(res.lse))


def _bits(t):
    return t.contiguous().view(torch.int16 if t.dtype == torch.bfloat16 else torch.int32)


@pytest.mark.parametrize("lengths,hq,hkv,dim,cap,splits", [
    ([2064], 16, 4, 256, 2112, 0), ([528], 16, 4, 256, 528, 0),
    ([0, 1, 257, 1000], 8, 2, 128, 1000, 0), ([0, 0, 0], 8, 2, 64, 2051, 0),
    ([2051, 1, 0, 1025], 32, 4, 256, 4096, 1), ([2051, 1, 0, 1025], 32, 2, 128, 4096, 6),
    ([3000, 17], 12, 4, 64, 4096, 0), ([4096] * 3, 16, 1, 256, 4096, 0),
    ([2064, 700], 16, 2, 256, 2112, 0), ([900, 0], 10, 2, 256, 1024, 0)])
def test_fused_decode_matches_two_launches(lengths, hq, hkv, dim, cap, splits):
    """The fused launch runs the partition kernel the two launches run for the same plan
    (the single-tile kernel for splits of one tile, the multi-tile kernel otherwise) and
    merges with lse_merge_kernel's arithmetic, so partials, LSEs and outputs are
    bit-identical; the split counters are zero again after every call."""
    g = to_gpu(make_case(lengths, hq, hkv, dim, seed=31, capacity=cap))
    res = allocate_matched_resources(DecodeSpec(len(lengths), hq, hkv, dim, cap), "cuda",
                                     num_splits=splits, fused=True)
    two = _two_kernel_resources(res)
    for _ in range(3):
        poison_workspace(res)
        poison_workspace(two)
        fused = matched_decode(*g, resources=res).clone()
        split = matched_decode(*g, resources=two).clone()
        torch.cuda.synchronize()
        assert torch.equal(_bits(res.lse), _bits(two.lse))
        assert torch.count_nonzero(res.counters) == 0
        assert torch.equal(_bits(fused), _bits(split))
        assert torch.equal(_bits(res.partials), _bits(two.partials))


def test_fused_counters_return_to_zero_across_graph_replays():
    case = make_case([2064], 16, 4, 256, seed=3, capacity=2112)
    g = to_gpu(case)
    res = allocate_matched_resources(DecodeSpec(1, 16, 4, 256, 2112), "cuda", fused=True)
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        for _ in range(3):
            matched_decode(*g, resources=res)
    torch.cuda.current_stream().wait_stream(stream)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for _ in range(8):
            out = matched_decode(*g, resources=res)
    expected = matched_decode(*g, resources=_two_kernel_resources(res)).clone()
    for _ in range(5):
        poison_workspace(res)
        graph.replay()
        torch.cuda.synchronize()
        assert torch.count_nonzero(res.counters) == 0
        assert torch.equal(_bits(out), _bits(expected))


def test_fixed_plan_contract():
    # reference tests/test_matched_splitkv.py:60-69.
    g = to_gpu(make_case([1, 2, 0], 8, 2, 256, capacity=2051))
    res = allocate_matched_resources(DecodeSpec(3, 8, 2, 256, 2051), "cuda")
    q, k, v, table, lengths = g
    with pytest.raises(ValueError, match="fixed batch"):
        matched_decode(q[:1], k, v, table[:1], lengths[:1], resources=res)
    with pytest.raises(ValueError, match="fixed batch"):
        matched_decode(q, k, v, table[:, :8], lengths, resources=res)
    with pytest.raises(ValueError, match="positive"):
        matched_decode(*g, resources=res, scale=0)
    with pytest.raises(ValueError, match="BF16"):
        matched_decode(q.float(), k, v, table, lengths, resources=res)
    bad = allocate_matched_resources(DecodeSpec(3, 8, 2, 256, 2051), "cuda", num_splits=2)
    bad.lse = bad.lse[:, :, :1]
    with pytest.raises(ValueError, match="workspace"):
        matched_decode(*g, resources=bad)


def test_cpu_reference_config_c1():
    # B=4, Hq=8, Hkv=2, D=128, lengths {0,1,257,1000}.
    case = make_case([0, 1, 257, 1000], 8, 2, 128, seed=1, capacity=1000)
    g, res, out = run(case, DecodeSpec(4, 8, 2, 128, 1000))
    check_all(case, g, res, out)
    assert torch.count_nonzero(out[0]) == 0


def _edge_lengths(rng, batch, maximum):
    lengths = rng.integers(1, maximum + 1, size=batch)
    lengths[rng.permutation(batch)[: batch // 4]] = 0
    special = [255, 256, 257, 511, 512, 513, 1023, 1024, 1025, 2047, 2048, 2049, maximum]
    lengths[batch // 4: batch // 4 + len(special)] = special
    return lengths.astype(np.int32)


@pytest.mark.parametrize("dim,hq,hkv", [(64, 16, 16), (256, 32, 4)])
@pytest.mark.parametrize("splits", [0, 3, 6])
def test_edge_coverage_config_c4(dim, hq, hkv, splits):
    rng = np.random.default_rng(404)
    lengths = _edge_lengths(rng, 128, 4096)
    case = make_case(list(lengths), hq, hkv, dim, seed=5, capacity=4096)
    g, res, out = run(case, DecodeSpec(128, hq, hkv, dim, 4096), num_splits=splits)
    check_all(case, g, res, out, where=f"D{dim} {hq}/{hkv} splits {res.plan.splits}")
    zero_rows = torch.from_numpy(lengths == 0).cuda()
    assert torch.count_nonzero(out[zero_rows]) == 0


@pytest.mark.parametrize("dim", [64, 128, 256])
@pytest.mark.parametrize("group", [1, 2, 3, 5, 6, 8, 12, 16])
def test_gqa_group_sizes(dim, group):
    hkv = 2
    case = make_case([0, 1, 300, 1025], hkv * group, hkv, dim, seed=group, capacity=1500)
    for splits in (0, 3):
        g, res, out = run(case, DecodeSpec(4, hkv * group, hkv, dim, 1500), num_splits=splits)
        check_all(case, g, res, out, where=f"G{group} D{dim} splits {splits}")


def test_custom_scale_and_strided_query():
    case = make_case([700, 1, 2000], 8, 2, 128, seed=11, capacity=2048)
    q, k, v, table, lengths = to_gpu(case)
    wide = torch.zeros((3, 10, 128), device="cuda", dtype=torch.bfloat16)
    wide[:, 1:9] = q
    strided = wide[:, 1:9]            # stride(0) = 1280, stride(1) = 128
    assert not strided.is_contiguous()
    res = allocate_matched_resources(DecodeSpec(3, 8, 2, 128, 2048), "cuda")
    poison_workspace(res)
    out = matched_decode(strided, k, v, table, lengths, resources=res, scale=0.0625)
    torch.cuda.synchronize()
    check_all(case, (q, k, v, table, lengths), res, out, scale=0.0625)


def test_long_single_split_reverse_walk():
    # One split over up to 32768 tokens: 256 tiles walked last-to-first.
    case = make_case([32768, 20000], 32, 8, 128, seed=3, capacity=32768)
    g, res, out = run(case, DecodeSpec(2, 32, 8, 128, 32768), num_splits=1)
    check_all(case, g, res, out)


def test_single_split_beyond_the_prefetched_table_window():
    # 160 pages in one partition: the first 128 table entries are fetched at
    # kernel entry, the rest are read as the reverse walk reaches them.
    case = make_case([40000, 33000, 256], 4, 1, 64, seed=8, capacity=40960)
    g, res, out = run(case, DecodeSpec(3, 4, 1, 64, 40960), num_splits=1)
    assert res.plan.tokens_per_split == 40960
    check_all(case, g, res, out)



@pytest.mark.parametrize("fused", [False, True])
def test_d256_tile_counts_of_the_loader_kernel(fused):
    """D=256 multi-tile splits run cols_loader_kernel, whose loader wavefronts issue
    and wait differently for one, two and more tiles: splits of 1 to 8 tiles (64
    tokens each), full and partial."""
    lengths = [1, 64, 65, 128, 130, 192, 200, 256, 300, 384, 450, 511, 512]
    case = make_case(lengths, 16, 4, 256, seed=41, capacity=512)
    g = to_gpu(case)
    res = allocate_matched_resources(DecodeSpec(len(lengths), 16, 4, 256, 512), "cuda",
                                     num_splits=1, fused=fused)
    assert res.plan.tokens_per_split == 512
    poison_workspace(res)
    out = matched_decode(*g, resources=res)
    torch.cuda.synchronize()
    check_all(case, g, res, out, where=f"fused={fused}")


@pytest.mark.parametrize("splits,tokens,lengths", [
    (1, 512, [1, 64, 65, 128, 130, 192, 200, 256, 300, 384, 450, 511, 512]),
    (3, 1024, [2064, 1, 1024, 1025, 2048, 3000, 3072]),
    (4, 2048, [8192, 6000, 100, 2049]),
])
def test_d256_partials_of_a_sequence_alone_and_in_a_batch(splits, tokens, lengths):
    """D=256 multi-tile partitions (cols_loader_kernel) of each sequence alone (B=1,
    every workgroup on a CU of its own) and as a row of a batch whose grid exceeds
    the CUs (two rounds, longest first): the same partial and LSE bits, with
    partial tiles, NaN-poisoned tails and several splits; the batch passes the
    oracle."""
    hq, hkv = 16, 4
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    batch = cus // (splits * hkv) + 1
    rows = (lengths * batch)[:batch]
    q, k, v, table, lens = make_case(rows, hq, hkv, 256, seed=77, capacity=splits * tokens)
    poison_tails(k, v, table, lens)
    case = (q, k, v, table, lens)
    g = to_gpu(case)

    def partition(qq, tt, ll):
        partials = torch.full((qq.shape[0], hq, splits, 256), float("nan"), device="cuda")
        lse = torch.full((qq.shape[0], hq, splits), float("nan"), device="cuda")
        _native.partition(qq, g[1], g[2], tt, ll, partials, lse, hkv, splits, tokens, 64,
                          256 ** -0.5)
        return partials, lse

    big_partials, big_lse = partition(g[0], g[3], g[4])
    for r in range(len(lengths)):
        one_partials, one_lse = partition(g[0][r:r + 1], g[3][r:r + 1], g[4][r:r + 1])
        torch.cuda.synchronize()
        where = f"length {rows[r]}, {splits} x {tokens}"
        assert torch.equal(one_partials.view(torch.int32), big_partials[r:r + 1].view(torch.int32)), where
        assert torch.equal(one_lse.view(torch.int32), big_lse[r:r + 1].view(torch.int32)), where
    lanes = min(1 << (splits - 1).bit_length(), 32)
    _, partials, lse, _, partial_bound = OM.matched_decode_with_bounds(*case, splits, tokens, 64,
                                                                       lanes)
    np.testing.assert_allclose(to_np(big_lse), lse, atol=2e-5, rtol=1e-6)
    assert_partials(big_partials, partials, partial_bound)


@pytest.mark.parametrize("dim,hq,hkv", [(64, 8, 2), (128, 16, 4), (256, 16, 4), (256, 12, 3)])
def test_single_tile_and_multi_tile_kernels_agree_on_one_tile(dim, hq, hkv):
    """A split holding one tile of tokens gives the same partial and LSE bits whether it
    runs the single-tile kernel (tokens_per_split == tile) or the loader kernel (a
    two-tile split whose second tile is past the sequence end): both compute scores,
    maxima, probabilities and denominators the same way and P V in the same k-step
    order."""
    tile = 16384 // dim
    lengths = [tile, tile - 1, 1, 0, tile // 2 + 3]
    q, k, v, table, lens = make_case(lengths, hq, hkv, dim, seed=61, capacity=2 * tile)
    poison_tails(k, v, table, lens)
    g = to_gpu((q, k, v, table, lens))
    out = {}
    for tokens in (tile, 2 * tile):
        partials = torch.full((len(lengths), hq, 1, dim), float("nan"), device="cuda")
        lse = torch.full((len(lengths), hq, 1), float("nan"), device="cuda")
        _native.partition(*g, partials, lse, hkv, 1, tokens, tile, dim ** -0.5)
        torch.cuda.synchronize()
        out[tokens] = (partials, lse)
    assert torch.equal(out[tile][1].view(torch.int32), out[2 * tile][1].view(torch.int32))
    assert torch.equal(out[tile][0].view(torch.int32), out[2 * tile][0].view(torch.int32))


@pytest.mark.parametrize("dim,hq,hkv,cap,splits", [(128, 32, 8, 2048, 8), (256, 16, 8, 1024, 8),
                                                   (64, 16, 8, 4096, 8), (256, 32, 4, 3000, 12)])
def test_walk_of_several_splits_per_workgroup(dim, hq, hkv, cap, splits):
    """Plans with more (split, kv head, sequence) workgroups than CUs run one resident round
    in which each workgroup walks several consecutive splits of its sequence.  Every split
    must keep its bits: each row of such a batch (8 sequences, splits x kv heads x 8 > 256
    workgroups) equals the same sequence run alone (one workgroup per split), partials, LSEs
    and output bit for bit, from NaN workspaces; and the batch passes the oracle's gate."""
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    batch = 8
    assert splits * hkv * batch > cus >= splits * hkv, "the batch must walk, one sequence not"
    tile = 16384 // dim
    part = -(-(-(-cap // tile)) // splits) * tile
    lengths = [0, 1, part - 1, part, part + 1, 3 * part + tile // 2, cap - 1, cap]
    case = make_case(lengths, hq, hkv, dim, seed=splits + dim, capacity=cap)
    poison_tails(*case[1:3], case[3], case[4])
    spec = DecodeSpec(batch, hq, hkv, dim, cap)
    g, res, out = run(case, spec, num_splits=splits)
    assert res.plan.splits == splits and res.plan.tokens_per_split == part
    check_all(case, g, res, out, where=f"walk D{dim} {hq}/{hkv} {splits}x{part}")
    q, k, v, table, lens = g
    for i in range(batch):
        alone = allocate_matched_resources(DecodeSpec(1, hq, hkv, dim, cap), "cuda",
                                           num_splits=splits)
        poison_workspace(alone)
        one = matched_decode(q[i:i + 1], k, v, table[i:i + 1], lens[i:i + 1], resources=alone)
        torch.cuda.synchronize()
        assert torch.equal(one.view(torch.int16), out[i:i + 1].view(torch.int16)), f"row {i}"
        assert torch.equal(alone.partials.view(torch.int32), res.partials[i:i + 1].view(torch.int32))
        assert torch.equal(alone.lse.view(torch.int32), res.lse[i:i + 1].view(torch.int32))
