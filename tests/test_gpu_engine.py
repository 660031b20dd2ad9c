"""A nano-vLLM-style engine loop over this operator: configure_model, prefill, decode
steps eager and from captured decode graphs with padded batch buckets.

Follows the overlay's call pattern (overlays/nano-vllm/nanovllm/layers/attention.py:61-82,
engine/model_runner.py:106-128 cache allocation, :179-195 decode metadata, :214-230
graph replay with slot_mapping -1 / context_lens 0 padding, :241-276 capture).
Decode outputs are checked against a float32 dense attention over the cache contents,
and graph replays against eager steps bit for bit (outputs and cache writes).
"""
from types import SimpleNamespace

import numpy as np
import pytest
import torch
from torch import nn

if not torch.cuda.is_available():
    pytest.skip("needs an MI355X GPU", allow_module_level=True)

from gpu_cases import assert_close_dense
from paged_decode.engine_attention import (Attention, DecodeTimings, decode_metadata,
                                           graph_batch_sizes, reset_context, set_context)
from paged_decode.integration import configure_model

pytestmark = pytest.mark.gpu

GEOMETRIES = [(16, 8, 128), (32, 4, 256), (16, 8, 128), (16, 16, 64)]
BLOCKS = 48


class Engine:
    """Minimal engine state: per-layer paged caches, sequences and their block tables."""

    def __init__(self, backend, max_num_seqs=8, max_model_len=2048, seed=0):
        self.gen = torch.Generator(device="cuda").manual_seed(seed)
        self.layers = nn.ModuleList(Attention(hq, d, d ** -0.5, hkv) for hq, hkv, d in GEOMETRIES)
        for layer in self.layers:
            shape = (BLOCKS, 256, layer.num_kv_heads, layer.head_dim)
            layer.k_cache = torch.full(shape, float("nan"), device="cuda", dtype=torch.bfloat16)
            layer.v_cache = torch.full(shape, float("nan"), device="cuda", dtype=torch.bfloat16)
        self.config = SimpleNamespace(decode_backend=backend, max_num_seqs=max_num_seqs,
                                      max_model_len=max_model_len, kvcache_block_size=256)
        configure_model(self.layers, self.config)
        rng = np.random.default_rng(seed)
        self.free = [int(b) for b in rng.permutation(BLOCKS)]
        self.tables, self.lens = [], []

    def qkv(self, layer, n):
        q = torch.randn((n, layer.num_heads, layer.head_dim), generator=self.gen, device="cuda")
        k = torch.randn((n, layer.num_kv_heads, layer.head_dim), generator=self.gen, device="cuda")
        v = torch.randn((n, layer.num_kv_heads, layer.head_dim), generator=self.gen, device="cuda")
        return q.bfloat16(), k.bfloat16(), v.bfloat16()

    def prefill(self, prompt_lens):
        slots, cu = [], [0]
        for n in prompt_lens:
            table = [self.free.pop() for _ in range((n + 255) // 256)]
            self.tables.append(table)
            self.lens.append(n)
            slots += [table[p // 256] * 256 + p % 256 for p in range(n)]
            cu.append(cu[-1] + n)
        cu_t = torch.tensor(cu, dtype=torch.int32, device="cuda")
        set_context(True, cu_t, cu_t, max(prompt_lens), max(prompt_lens),
                    torch.tensor(slots, dtype=torch.int32, device="cuda"))
        for layer in self.layers:
            out = layer(*self.qkv(layer, cu[-1]))
            assert out.shape == (cu[-1], layer.num_heads, layer.head_dim)
        reset_context()

    def grow(self):
        """One more token per sequence (a new block when the last one is full)."""
        for i in range(len(self.lens)):
            if self.lens[i] % 256 == 0:
                self.tables[i].append(self.free.pop())
            self.lens[i] += 1


def dense(layer, q, tables, lens):
    """float32 attention of each sequence's query over its cached tokens."""
    out = torch.zeros((len(lens), layer.num_heads, layer.head_dim), device="cuda")
    group = layer.num_heads // layer.num_kv_heads
    for b, (table, n) in enumerate(zip(tables, lens)):
        pos = torch.arange(n, device="cuda")
        blocks = torch.tensor(table, device="cuda")[pos // 256]
        keys = layer.k_cache[blocks, pos % 256].float().repeat_interleave(group, 1).transpose(0, 1)
        vals = layer.v_cache[blocks, pos % 256].float().repeat_interleave(group, 1).transpose(0, 1)
        s = torch.matmul(keys, q[b].float().unsqueeze(-1)).squeeze(-1) * layer.scale
        out[b] = torch.matmul(s.softmax(-1).unsqueeze(1), vals).squeeze(1)
    return out


@pytest.mark.parametrize("backend", ["hip_base", "hip_splitk", "triton_splitk"])
def test_eager_decode_steps_match_dense_attention(backend):
    eng = Engine(backend)
    eng.prefill([300, 17, 600, 256])
    for _ in range(3):
        eng.grow()
        slots, lens, tables = decode_metadata(eng.tables, eng.lens)
        set_context(False, slot_mapping=slots, context_lens=lens, block_tables=tables)
        for layer in eng.layers:
            q, k, v = eng.qkv(layer, len(eng.lens))
            out = layer(q, k, v)
            assert out.shape == (len(eng.lens), 1, layer.num_heads, layer.head_dim)
            assert_close_dense(out[:, 0], dense(layer, q, eng.tables, eng.lens))
        reset_context()


@pytest.mark.parametrize("backend", ["hip_base", "hip_splitk"])
def test_captured_decode_buckets_equal_eager_steps(backend):
    eng = Engine(backend, max_num_seqs=8)
    eng.prefill([300, 17, 600])
    eng.grow()
    live = len(eng.lens)
    bucket = next(b for b in graph_batch_sizes(eng.config.max_num_seqs) if b >= live)
    max_blocks = (eng.config.max_model_len + 255) // 256
    gv = dict(slot_mapping=torch.full((8,), -1, dtype=torch.int32, device="cuda"),
              context_lens=torch.zeros(8, dtype=torch.int32, device="cuda"),
              block_tables=torch.zeros((8, max_blocks), dtype=torch.int32, device="cuda"))
    inputs = [tuple(torch.zeros((8, *t.shape[1:]), dtype=torch.bfloat16, device="cuda")
                    for t in eng.qkv(layer, 1)) for layer in eng.layers]
    # Layers of one geometry share one borrowed output buffer, so each layer's output
    # is consumed (copied, as a projection would) before the next layer runs.
    outputs = [torch.zeros((8, 1, l.num_heads, l.head_dim), dtype=torch.bfloat16, device="cuda")
               for l in eng.layers]

    def step(bs):
        for i, layer in enumerate(eng.layers):
            q, k, v = (t[:bs] for t in inputs[i])
            outputs[i][:bs].copy_(layer(q, k, v))

    set_context(False, slot_mapping=gv["slot_mapping"][:bucket],
                context_lens=gv["context_lens"][:bucket], block_tables=gv["block_tables"][:bucket])
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        step(bucket)                               # warmup (all slots -1, lengths 0)
    torch.cuda.current_stream().wait_stream(stream)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step(bucket)
    reset_context()

    for _ in range(2):
        step_inputs = [eng.qkv(layer, live) for layer in eng.layers]
        slots, lens, tables = decode_metadata(eng.tables, eng.lens)
        caches = [(l.k_cache.clone(), l.v_cache.clone()) for l in eng.layers]
        # eager step
        set_context(False, slot_mapping=slots, context_lens=lens, block_tables=tables)
        eager = [layer(*x).clone() for layer, x in zip(eng.layers, step_inputs)]
        reset_context()
        after = [(l.k_cache.clone(), l.v_cache.clone()) for l in eng.layers]
        for layer, (kc, vc) in zip(eng.layers, caches):
            layer.k_cache.copy_(kc)
            layer.v_cache.copy_(vc)
        # graph replay with the engine's padding of unused rows
        for buf, x in zip(inputs, step_inputs):
            for dst, src in zip(buf, x):
                dst[:live] = src
        gv["slot_mapping"].fill_(-1)
        gv["slot_mapping"][:live] = slots
        gv["context_lens"].zero_()
        gv["context_lens"][:live] = lens
        gv["block_tables"][:live, :tables.shape[1]] = tables
        graph.replay()
        torch.cuda.synchronize()
        for i, layer in enumerate(eng.layers):
            assert torch.equal(outputs[i][:live].view(torch.int16), eager[i].view(torch.int16))
            assert torch.count_nonzero(outputs[i][live:bucket]) == 0    # padded rows: length 0
            assert torch.equal(layer.k_cache.view(torch.int16), after[i][0].view(torch.int16))
            assert torch.equal(layer.v_cache.view(torch.int16), after[i][1].view(torch.int16))
            assert_close_dense(eager[i][:, 0], dense(layer, step_inputs[i][0], eng.tables, eng.lens))
        eng.grow()


def test_decode_timings_of_eager_steps_and_graph_replays():
    """DecodeTimings records one interval per decode step, eager or replayed, with its
    batch; prefill steps and disabled timing record nothing."""
    eng = Engine("hip_splitk")
    timings = DecodeTimings()
    timings.run(lambda: eng.prefill([300, 17]), 2, is_prefill=True)
    eng.grow()
    slots, lens, tables = decode_metadata(eng.tables, eng.lens)
    set_context(False, slot_mapping=slots, context_lens=lens, block_tables=tables)
    inputs = [eng.qkv(layer, len(eng.lens)) for layer in eng.layers]
    step = lambda: [layer(*x).clone() for layer, x in zip(eng.layers, inputs)]
    eager = timings.run(step, len(eng.lens))
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        step()
    torch.cuda.current_stream().wait_stream(stream)
    # Layers of one geometry share a borrowed output buffer: each output is copied out.
    outs = [torch.empty_like(e) for e in eager]
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for dst, layer, x in zip(outs, eng.layers, inputs):
            dst.copy_(layer(*x))
    for _ in range(3):
        timings.run(graph.replay, len(eng.lens))
    timings.enabled = False
    timings.run(graph.replay, len(eng.lens))
    reset_context()
    got = timings.intervals()
    assert [g["batch"] for g in got] == [2, 2, 2, 2]
    assert all(g["milliseconds"] > 0 for g in got)
    for a, b in zip(eager, outs):
        assert torch.equal(a.view(torch.int16), b.view(torch.int16))
    timings.clear()
    assert timings.intervals() == []
