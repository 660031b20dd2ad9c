"""The reference's D256 replay correctness matrix (tools/resident_experiment.py:30-80).

Three GQA geometries (Hq, Hkv) in {(8, 8), (32, 8), (16, 1)} at D 256, batch 8,
capacity 2051, with the planner's split count and with one explicit split.  A
graph is captured after warm-up at the first length state, then replayed through
four states:
* the initial lengths {0, 1, 255, 256, 257, 1023, 1024, 1025}, with table entries
  past each sequence's live pages set to -1 and the slots past its length in its
  last page NaN;
* three more length states, with the page table reversed on odd steps, and new
  Q, K and V each time (the last state is all zero lengths).
At every state, for the two-launch and the single-launch (fused) decode, with the
output and workspaces NaN-poisoned before every replay and eager call:
* the replayed output equals an eager call bit for bit;
* it is within the oracle's one-ulp gate and within 2e-2 of the float32 dense
  reference (max-abs and RMSE are recorded for the run's parity summary);
* the fused and two-launch paths agree bit for bit (output, partials, LSEs);
* the all-zero state gives exact zeros.
The reference also compares against FlashAttention's paged decode bit for bit;
flash-attn does not exist for this GPU, so that comparison has no counterpart.
"""
import pytest
import torch

if not torch.cuda.is_available():
    pytest.skip("needs an MI355X GPU", allow_module_level=True)

from gpu_cases import (assert_close_dense, assert_within_one_ulp, poison_workspace, to_np,
                       torch_dense)
from oracle import matched as OM
from paged_decode.matched_splitkv import allocate_matched_resources, matched_decode
from paged_decode.spec import DecodeSpec

pytestmark = pytest.mark.gpu

INITIAL = [0, 1, 255, 256, 257, 1023, 1024, 1025]
STATES = [INITIAL, [257, 1025, 0, 2051, 1, 256, 1024, 255], [1, 0, 1025, 0, 2051, 257, 256, 1],
          [0] * 8]


def capture(fn):
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        for _ in range(3):
            fn()
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = fn()
    return graph, out


@pytest.mark.parametrize("splits", [0, 1])
@pytest.mark.parametrize("hq,hkv", [(8, 8), (32, 8), (16, 1)])
def test_replay_matrix(hq, hkv, splits):
    torch.manual_seed(123)
    spec = DecodeSpec(8, hq, hkv, 256, 2051)
    width = spec.table_width
    q = torch.randn(8, hq, 256, device="cuda", dtype=torch.bfloat16)
    k = torch.randn(8 * width, 256, hkv, 256, device="cuda", dtype=torch.bfloat16)
    v = torch.randn_like(k)
    table = torch.randperm(8 * width, device="cuda").int().view(8, width)
    lengths = torch.tensor(INITIAL, device="cuda", dtype=torch.int32)
    original = table.clone()
    for row, n in enumerate(INITIAL):
        table[row, (n + 255) // 256:] = -1
        if n % 256:
            page = int(original[row, n // 256])
            k[page, n % 256:] = float("nan")
            v[page, n % 256:] = float("nan")
    tensors = (q, k, v, table, lengths)
    paths = {"two_launch": allocate_matched_resources(spec, "cuda", num_splits=splits),
             "fused": allocate_matched_resources(spec, "cuda", num_splits=splits, fused=True)}
    plan = paths["two_launch"].plan
    graphs = {name: capture(lambda r=res: matched_decode(*tensors, resources=r))
              for name, res in paths.items()}
    for step, state in enumerate(STATES):
        if step:
            table.copy_(original.flip(1) if step % 2 else original)
            lengths.copy_(torch.tensor(state, dtype=torch.int32, device="cuda"))
            q.normal_()
            k.normal_()
            v.normal_()
        dense = torch_dense(*tensors)
        host = (to_np(q), to_np(k), to_np(v), table.cpu().numpy(), lengths.cpu().numpy())
        expected, _, _, bound, _, counts = OM.matched_decode_with_bounds(
            *host, plan.splits, plan.tokens_per_split, plan.tile_tokens, plan.lse_lanes,
            counts=True)
        values = {}
        for name, res in paths.items():
            graph, out = graphs[name]
            for _ in range(3):
                poison_workspace(res)
                graph.replay()
            torch.cuda.synchronize()
            replayed = out.clone()
            saved = (replayed, res.partials.clone(), res.lse.clone())
            poison_workspace(res)
            eager = matched_decode(*tensors, resources=res).clone()
            where = f"Hq {hq} Hkv {hkv} splits {plan.splits} step {step} {name}"
            assert torch.equal(replayed.view(torch.int16), eager.view(torch.int16)), where
            assert_close_dense(replayed, dense, where)
            assert_within_one_ulp(replayed, expected, where, bound, counts)
            if not any(state):
                assert torch.count_nonzero(replayed) == 0, where
            values[name] = saved
        for a, b in zip(values["fused"], values["two_launch"]):
            bits = torch.int32 if a.dtype == torch.float32 else torch.int16
            assert torch.equal(a.view(bits), b.view(bits)), f"step {step}: fused != two launches"
