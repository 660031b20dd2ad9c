"""Batch order of the multi-tile kernels, on the GPU.

With more workgroups than CUs, the multi-tile kernel (cols_loader_kernel, one workgroup
per CU) hands the grid's batch rows to the sequences in order of length
(ordered_sequence in pd_device.h): longest first when the grid runs in two to four
rounds; past four rounds the batch keeps its order.  Which workgroup runs an item must not change a bit of the
result.  Each case runs a batch large enough to switch the ordering on (the mode named
is the one a 256-CU device takes) and compares every output row, bit for bit, with the
same sequence run alone (batch 1, where the order is the identity), under the same plan.
Lengths include zeros, ties and page boundaries; the unused pool holds NaN.
"""
import numpy as np
import pytest
import torch

if not torch.cuda.is_available():
    pytest.skip("needs an MI355X GPU", allow_module_level=True)

from gpu_cases import assert_close_dense, pooled_case, torch_dense
from paged_decode.matched_splitkv import allocate_matched_resources, matched_decode
from paged_decode.runtime import allocate_resources, paged_decode
from paged_decode.spec import DecodeSpec

pytestmark = pytest.mark.gpu


def _bits(t):
    return t.contiguous().view(torch.int16)


def _lengths(batch, capacity, seed):
    rng = np.random.default_rng(seed)
    lengths = rng.integers(1, capacity + 1, size=batch)
    lengths[rng.permutation(batch)[: batch // 8]] = 0
    ties = rng.permutation(batch)[: batch // 4]
    lengths[ties] = lengths[ties[0]]                 # a quarter of the batch ties
    special = [1, 255, 256, 257, capacity - 1, capacity]
    lengths[:len(special)] = special
    return lengths.astype(np.int32)


def _one(g, b):
    q, k, v, table, lens = g
    return q[b:b + 1], k, v, table[b:b + 1], lens[b:b + 1]


def _walk(res):
    """paged_decode resources without the small-batch chunk workspace: every call walks."""
    res.chunk_maxima = res.chunk_denoms = res.chunk_accums = None
    return res


def _check_rows(full, g, alone):
    for b in range(full.shape[0]):
        out = alone(_one(g, b))
        assert torch.equal(_bits(out[0]), _bits(full[b])), f"sequence {b}"


# (dim, hq, hkv, batch, capacity): mode on 256 CUs for one split per sequence
MATCHED = [
    (128, 32, 8, 64, 2048),    # 512 workgroups, two rounds: longest first
    (128, 8, 8, 48, 2048),     # 384 workgroups, one and a half rounds: longest first
    (256, 32, 4, 128, 2048),   # 512 workgroups, one per CU (cols_loader_kernel): longest first
    (64, 16, 16, 128, 1024),   # 2048 workgroups, past four rounds: as given
    (128, 16, 4, 256, 512),    # 1024 workgroups, the largest batch that is ranked
    (128, 8, 8, 257, 512),     # 2056 workgroups, one sequence too many: as given
]


@pytest.mark.parametrize("dim,hq,hkv,batch,capacity", MATCHED)
def test_matched_rows_do_not_depend_on_the_batch_order(dim, hq, hkv, batch, capacity):
    lengths = _lengths(batch, capacity, seed=dim + batch)
    g = pooled_case(lengths, hq, hkv, dim, capacity, pool_pages=batch * capacity // 256 + 64,
                    seed=batch)
    res = allocate_matched_resources(DecodeSpec(batch, hq, hkv, dim, capacity), "cuda",
                                     num_splits=1)
    assert res.plan.tokens_per_split > res.plan.tile_tokens   # the multi-tile kernels
    full = matched_decode(*g, resources=res).clone()
    assert_close_dense(full, torch_dense(*g))
    single = allocate_matched_resources(DecodeSpec(1, hq, hkv, dim, capacity), "cuda",
                                        num_splits=1)
    assert single.plan.tokens_per_split == res.plan.tokens_per_split
    _check_rows(full, g, lambda c: matched_decode(*c, resources=single))


def test_two_sequences_over_many_splits():
    """64 splits x 4 kv heads x 2 sequences = 512 workgroups in two rounds: longest first."""
    dim, hq, hkv, capacity = 256, 16, 4, 8192
    lengths = np.array([8192, 3000], dtype=np.int32)
    g = pooled_case(lengths, hq, hkv, dim, capacity, pool_pages=96, seed=2)
    res = allocate_matched_resources(DecodeSpec(2, hq, hkv, dim, capacity), "cuda",
                                     num_splits=64)
    assert res.plan.tokens_per_split > res.plan.tile_tokens
    full = matched_decode(*g, resources=res).clone()
    assert_close_dense(full, torch_dense(*g))
    single = allocate_matched_resources(DecodeSpec(1, hq, hkv, dim, capacity), "cuda",
                                        num_splits=64)
    _check_rows(full, g, lambda c: matched_decode(*c, resources=single))


def test_fused_matched_rows_do_not_depend_on_the_batch_order():
    dim, hq, hkv, batch, capacity = 256, 16, 4, 64, 2048
    lengths = _lengths(batch, capacity, seed=7)
    g = pooled_case(lengths, hq, hkv, dim, capacity, pool_pages=batch * 8 + 64, seed=7)
    # 2 splits x 4 kv heads x 64 sequences = 512 workgroups in two rounds: longest first
    res = allocate_matched_resources(DecodeSpec(batch, hq, hkv, dim, capacity), "cuda",
                                     num_splits=2, fused=True)
    full = matched_decode(*g, resources=res).clone()
    single = allocate_matched_resources(DecodeSpec(1, hq, hkv, dim, capacity), "cuda",
                                        num_splits=2)
    _check_rows(full, g, lambda c: matched_decode(*c, resources=single))


@pytest.mark.parametrize("backend", ["hip_base", "hip_splitk"])
@pytest.mark.parametrize("dim,hq,hkv,batch,capacity", [
    (256, 32, 4, 128, 2048),   # 512 workgroups, one per CU, in two rounds: longest first
    (64, 16, 16, 128, 2048),   # four kv heads per workgroup: 512 workgroups, longest first
    (64, 32, 8, 64, 2048),     # four kv heads of 4 query heads: 128 workgroups, one per CU
    (64, 12, 6, 128, 2048),    # kv-head pairs (6 kv heads): 384 workgroups, longest first
    (128, 32, 8, 40, 2048),    # 320 workgroups, one and a quarter rounds: longest first
    (128, 64, 2, 128, 1024),   # 32-head groups in two 16-head slices: 512 workgroups
])
def test_paged_rows_do_not_depend_on_the_batch_order(backend, dim, hq, hkv, batch, capacity):
    lengths = _lengths(batch, capacity, seed=batch + hkv)
    g = pooled_case(lengths, hq, hkv, dim, capacity, pool_pages=batch * capacity // 256 + 64,
                    seed=hkv)
    # Both calls take the walk (no chunk workspace): the batch of one would take the
    # small-batch chunks otherwise, whose float32 rounding differs.
    res = _walk(allocate_resources(DecodeSpec(batch, hq, hkv, dim, capacity), "cuda", backend))
    full = paged_decode(*g, resources=res, backend=backend).clone()
    assert_close_dense(full, torch_dense(*g))
    single = _walk(allocate_resources(DecodeSpec(1, hq, hkv, dim, capacity), "cuda", backend))
    _check_rows(full, g, lambda c: paged_decode(*c, resources=single, backend=backend))


CAPTURE_FIRST = r"""
import sys
sys.path[:0] = {paths!r}
import torch
from gpu_cases import pooled_case
from paged_decode.matched_splitkv import allocate_matched_resources, matched_decode
from paged_decode.spec import DecodeSpec
import numpy as np
lengths = np.random.default_rng(1).integers(0, 2049, size=64).astype(np.int32)
g = pooled_case(lengths, 32, 8, 128, 2048, pool_pages=600, seed=1)
res = allocate_matched_resources(DecodeSpec(64, 32, 8, 128, 2048), "cuda", num_splits=1)
stream = torch.cuda.Stream()
stream.wait_stream(torch.cuda.current_stream())
graph = torch.cuda.CUDAGraph()
with torch.cuda.graph(graph, stream=stream):    # the library's first launch in this process
    out = matched_decode(*g, resources=res)
graph.replay()
torch.cuda.synchronize()
captured = out.clone()
eager = matched_decode(*g, resources=res).clone()
assert torch.equal(captured.view(torch.int16), eager.view(torch.int16))
print("capture-first ok")
"""


def test_first_launch_of_the_process_under_graph_capture():
    """The launcher queries the CU count on its first ordered launch; in a fresh process
    whose first library call is captured into a graph, the capture must succeed and its
    replay equal the eager call."""
    import os
    import subprocess
    import sys
    here = os.path.dirname(os.path.abspath(__file__))
    root = os.path.dirname(here)
    paths = [here, root, os.path.join(root, "paged-decode-lab_amd")]
    res = subprocess.run([sys.executable, "-c", CAPTURE_FIRST.format(paths=paths)],
                         capture_output=True, text=True, timeout=300)
    assert res.returncode == 0, res.stderr[-3000:]
    assert "capture-first ok" in res.stdout


@pytest.mark.parametrize("backend", ["matched", "hip_base", "hip_splitk"])
def test_strided_query_rows_in_an_ordered_batch(backend):
    """Q as a strided view (head stride 2D, row stride 2 Hq D) in an ordered batch gives the
    same bits as contiguous Q: the permuted row index addresses Q through its strides."""
    dim, hq, hkv, batch, capacity = 128, 32, 8, 64, 2048
    lengths = _lengths(batch, capacity, seed=11)
    q, k, v, table, lens = pooled_case(lengths, hq, hkv, dim, capacity,
                                       pool_pages=batch * 8 + 64, seed=11)
    wide = torch.zeros((batch, hq, 2 * dim), dtype=q.dtype, device=q.device)
    wide[..., :dim] = q
    strided = wide[..., :dim]
    assert not strided.is_contiguous()
    spec = DecodeSpec(batch, hq, hkv, dim, capacity)
    if backend == "matched":
        res = allocate_matched_resources(spec, "cuda", num_splits=1)
        call = lambda qq: matched_decode(qq, k, v, table, lens, resources=res).clone()
    else:
        res = allocate_resources(spec, "cuda", backend)
        call = lambda qq: paged_decode(qq, k, v, table, lens, resources=res,
                                       backend=backend).clone()
    assert torch.equal(_bits(call(strided)), _bits(call(q)))
