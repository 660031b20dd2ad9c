"""pd_matched_decode_noalloc against pd_matched_decode, through the C ABI.

The allocation-free entry point keeps its split workspace in the library's
static device scratch.  Its output must equal pd_matched_decode's (which takes
the workspace as arguments) bit for bit, on consecutive calls of different
sizes that share the scratch, eagerly and replayed from a hipGraph.
"""
import pytest
import torch

if not torch.cuda.is_available():
    pytest.skip("needs an MI355X GPU", allow_module_level=True)

from cases import make_case, poison_tails
from gpu_cases import to_gpu
from paged_decode import _native
from paged_decode.matched_splitkv import allocate_matched_resources
from paged_decode.spec import DecodeSpec

pytestmark = pytest.mark.gpu


def reference_call(g, spec, num_splits=0):
    """pd_matched_decode with its own workspace; returns (out, plan)."""
    res = allocate_matched_resources(spec, "cuda", num_splits=num_splits, fused=True)
    q, k, v, table, lens = g
    plan = res.plan
    _native.matched_decode(q, k, v, table, lens, res.partials, res.lse, res.counters, res.out,
                           spec.num_kv_heads, plan.splits, plan.tokens_per_split,
                           plan.tile_tokens, spec.head_dim ** -0.5)
    return res.out.clone(), plan


def noalloc_call(g, spec, plan, out):
    q, k, v, table, lens = g
    _native.matched_decode_noalloc(q, k, v, table, lens, out, spec.num_kv_heads, plan.splits,
                                   plan.tokens_per_split, plan.tile_tokens,
                                   spec.head_dim ** -0.5)


CASES = [
    # (lengths, Hq, Hkv, D, capacity, explicit splits): the benchmark's D256 GQA shape
    # with four sequences, then a smaller one (fewer rows, fewer splits, D 128), then
    # eight sequences whose plan (12 splits of 3 tiles, 384 workgroups) the partition
    # walks two splits per workgroup, against pd_matched_decode's one launch, which
    # runs one workgroup per split; last, one split of 33 tiles, whose output the
    # allocation-free partition writes itself.
    ([2064, 0, 1000, 1], 16, 4, 256, 2112, 0),
    ([257, 0], 8, 2, 128, 600, 0),
    ([2064, 0, 1000, 2064, 1, 2064, 1500, 192], 16, 4, 256, 2112, 0),
    # a plan of one split of 33 tiles: the partition writes the output, no merge runs
    ([2064, 0, 700], 16, 4, 256, 2112, 1),
]


def test_two_calls_in_a_row_match_pd_matched_decode():
    outs = []
    for lengths, hq, hkv, dim, cap, splits in CASES:
        print(f"noalloc case B={len(lengths)} Hq={hq} Hkv={hkv} D={dim} cap={cap}", flush=True)
        case = make_case(lengths, hq, hkv, dim, seed=len(lengths), capacity=cap)
        poison_tails(*case[1:3], case[3], case[4])
        g = to_gpu(case)
        spec = DecodeSpec(len(lengths), hq, hkv, dim, cap)
        expected, plan = reference_call(g, spec, splits)
        out = torch.full_like(expected, float("nan"))
        noalloc_call(g, spec, plan, out)
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), expected.view(torch.int16)), \
            f"B={len(lengths)} D={dim}: differs from pd_matched_decode"
        assert not out[lengths.index(0)].any(), "a zero-length row is not exactly zero"
        outs.append(out)
    # The first call's output is untouched by the second call, which reused the scratch.
    assert outs[0].isfinite().all()


def test_graph_replay_equals_eager():
    lengths, hq, hkv, dim, cap, _ = CASES[0]
    spec = DecodeSpec(len(lengths), hq, hkv, dim, cap)
    case = make_case(lengths, hq, hkv, dim, seed=3, capacity=cap)
    g = to_gpu(case)
    expected, plan = reference_call(g, spec)
    out = torch.empty_like(expected)
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        noalloc_call(g, spec, plan, out)
    torch.cuda.current_stream().wait_stream(stream)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        noalloc_call(g, spec, plan, out)
    for replay in range(3):
        out.zero_()
        # Eager work on the same scratch between replays (a different, smaller call).
        small = CASES[1]
        sspec = DecodeSpec(len(small[0]), *small[1:5])
        sg = to_gpu(make_case(small[0], *small[1:4], seed=replay, capacity=small[4]))
        sexp, splan = reference_call(sg, sspec)
        sout = torch.empty_like(sexp)
        noalloc_call(sg, sspec, splan, sout)
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(sout.view(torch.int16), sexp.view(torch.int16))
        assert torch.equal(out.view(torch.int16), expected.view(torch.int16)), f"replay {replay}"


def test_oversized_workspace_is_rejected():
    q = torch.zeros((64, 32, 256), device="cuda", dtype=torch.bfloat16)
    kv = torch.zeros((1, 256, 8, 256), device="cuda", dtype=torch.bfloat16)
    table = torch.zeros((64, 128), device="cuda", dtype=torch.int32)
    lens = torch.zeros((64,), device="cuda", dtype=torch.int32)
    out = torch.empty_like(q)
    # 64 * 32 * 32 splits * 257 floats = 67 MB > 16 MiB.
    with pytest.raises(ValueError, match="static scratch"):
        _native.matched_decode_noalloc(q, kv, kv, table, lens, out, 8, 32, 1024, 64, 0.0625)


NOALLOC_CAPTURE_FIRST = r"""
import sys
sys.path[:0] = {paths!r}
import torch
from cases import make_case
from gpu_cases import to_gpu
from paged_decode import _native
from paged_decode.matched_splitkv import allocate_matched_resources
from paged_decode.spec import DecodeSpec
lengths, hq, hkv, dim, cap = [2064, 0, 1000, 1], 16, 4, 256, 2112
spec = DecodeSpec(len(lengths), hq, hkv, dim, cap)
g = to_gpu(make_case(lengths, hq, hkv, dim, seed=5, capacity=cap))
plan = allocate_matched_resources(spec, "cuda").plan   # host planner and buffers only
q, k, v, table, lens = g
out = torch.full((len(lengths), hq, dim), float("nan"), device="cuda", dtype=torch.bfloat16)
torch.cuda.synchronize()
stream = torch.cuda.Stream()
stream.wait_stream(torch.cuda.current_stream())
graph = torch.cuda.CUDAGraph()
with torch.cuda.graph(graph, stream=stream):    # the library's first launch in this process
    _native.matched_decode_noalloc(q, k, v, table, lens, out, hkv, plan.splits,
                                   plan.tokens_per_split, plan.tile_tokens, dim ** -0.5)
graph.replay()
torch.cuda.synchronize()
captured = out.clone()
out.fill_(float("nan"))
_native.matched_decode_noalloc(q, k, v, table, lens, out, hkv, plan.splits,
                               plan.tokens_per_split, plan.tile_tokens, dim ** -0.5)
torch.cuda.synchronize()
assert torch.equal(captured.view(torch.int16), out.view(torch.int16)), "replay != eager"
assert not captured[1].any(), "zero-length row is not exactly zero"
print("noalloc capture-first ok")
"""


def test_first_call_of_the_process_under_graph_capture():
    """A fresh process whose first library launch is pd_matched_decode_noalloc inside a
    graph capture: the per-device scratch lookup then happens during the capture, which
    must still succeed, and the replay must equal an eager call bit for bit."""
    import os
    import subprocess
    import sys
    here = os.path.dirname(os.path.abspath(__file__))
    root = os.path.dirname(here)
    paths = [here, root, os.path.join(root, "paged-decode-lab_amd")]
    print("noalloc capture-first subprocess: B=4 Hq=16 Hkv=4 D=256", flush=True)
    res = subprocess.run([sys.executable, "-c", NOALLOC_CAPTURE_FIRST.format(paths=paths)],
                         capture_output=True, text=True, timeout=300)
    assert res.returncode == 0, res.stderr[-3000:]
    assert "noalloc capture-first ok" in res.stdout
