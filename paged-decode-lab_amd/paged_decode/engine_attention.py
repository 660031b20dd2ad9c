"""The attention layer of a nano-vLLM-style engine, with the decode step on this operator.

Restates the overlay's ``Attention`` module and the engine context it reads
(overlays/nano-vllm/nanovllm/layers/attention.py:43-82; the context fields are the ones
ModelRunner.prepare_prefill / prepare_decode set, engine/model_runner.py:136-195):

* every forward first writes the step's new K/V rows into the paged cache through
  ``context.slot_mapping`` (``store_kvcache``, a HIP kernel; slot -1 is skipped, which is
  how padded rows of a captured decode graph write nothing);
* a decode step calls ``paged_decode`` on the layer's cache with the engine's block
  tables (-1 padded in eager mode) and context lengths, using the ``decode_backend`` and
  ``decode_resources`` that ``integration.configure_model`` attached;
* prefill is not part of this operator: it runs a float32 PyTorch causal attention per
  sequence (the overlay uses flash-attn's varlen kernel there, which does not exist for
  this GPU), reading the cache through the block tables when a prefix is cached.

``decode_backend == "flash_attn"`` (the overlay's default before ``configure_model``)
has no kernel on this platform and raises.
"""
from dataclasses import dataclass

import torch
from torch import nn

from .kv_write import store_kvcache
from .runtime import paged_decode


@dataclass
class Context:
    is_prefill: bool = False
    cu_seqlens_q: torch.Tensor | None = None
    cu_seqlens_k: torch.Tensor | None = None
    max_seqlen_q: int = 0
    max_seqlen_k: int = 0
    slot_mapping: torch.Tensor | None = None
    context_lens: torch.Tensor | None = None
    block_tables: torch.Tensor | None = None


_CONTEXT = Context()


def get_context():
    return _CONTEXT


def set_context(is_prefill, cu_seqlens_q=None, cu_seqlens_k=None, max_seqlen_q=0,
                max_seqlen_k=0, slot_mapping=None, context_lens=None, block_tables=None):
    global _CONTEXT
    _CONTEXT = Context(is_prefill, cu_seqlens_q, cu_seqlens_k, max_seqlen_q, max_seqlen_k,
                       slot_mapping, context_lens, block_tables)


def reset_context():
    global _CONTEXT
    _CONTEXT = Context()


def decode_metadata(block_tables, seq_lens, block_size=256, device="cuda"):
    """Decode-step context tensors as ModelRunner.prepare_decode builds them.

    ``block_tables``: one list of physical blocks per sequence; ``seq_lens``: tokens per
    sequence including the one being decoded.  Returns (slot_mapping, context_lens,
    block_tables) with tables padded by -1 to the longest row
    (engine/model_runner.py:130-134,179-195).
    """
    slots, lens = [], []
    for table, n in zip(block_tables, seq_lens):
        last_block_tokens = n - (len(table) - 1) * block_size
        slots.append(table[-1] * block_size + last_block_tokens - 1)
        lens.append(n)
    width = max(len(t) for t in block_tables)
    padded = [list(t) + [-1] * (width - len(t)) for t in block_tables]
    return (torch.tensor(slots, dtype=torch.int32, device=device),
            torch.tensor(lens, dtype=torch.int32, device=device),
            torch.tensor(padded, dtype=torch.int32, device=device))


class DecodeTimings:
    """Per-step decode intervals of an engine, as the overlay's ModelRunner keeps them
    when ``Config.record_decode_timings`` is set (engine/model_runner.py:203-211): a pair
    of timing events around each decode step's model call (eager or graph replay) and
    the step's batch.  Prefill steps, and every step while ``enabled`` is false, run
    untimed.  ``intervals()`` reads them back in the form tools/benchmark_engine.py:66-67
    reports, ``[{"milliseconds": ..., "batch": ...}]``; reading synchronizes on the last
    event, so call it after the generation, not inside one."""

    def __init__(self, enabled=True):
        self.enabled = enabled
        self.records = []

    def run(self, step, batch, is_prefill=False):
        """``step()`` (one model call), timed when it is a decode step and timing is on."""
        if is_prefill or not self.enabled:
            return step()
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        start.record()
        result = step()
        end.record()
        self.records.append((start, end, int(batch)))
        return result

    def intervals(self):
        if self.records:
            self.records[-1][1].synchronize()
        return [{"milliseconds": a.elapsed_time(b), "batch": n} for a, b, n in self.records]

    def clear(self):
        self.records.clear()


def graph_batch_sizes(max_num_seqs):
    """Decode graph buckets of the engine: 1, 2, 4, 8, then every 16 up to the maximum
    (engine/model_runner.py:250-251)."""
    max_bs = min(max_num_seqs, 512)
    return sorted({b for b in [1, 2, 4, 8] + list(range(16, max_bs + 1, 16)) if b <= max_bs}
                  | {max_bs})


class Attention(nn.Module):

    def __init__(self, num_heads, head_dim, scale, num_kv_heads):
        super().__init__()
        self.num_heads = num_heads
        self.head_dim = head_dim
        self.scale = scale
        self.num_kv_heads = num_kv_heads
        self.k_cache = self.v_cache = torch.tensor([])
        self.decode_backend = "flash_attn"
        self.decode_resources = None

    def forward(self, q, k, v):
        """q [N, Hq, D], k/v [N, Hkv, D] of this step's tokens; returns [N, Hq, D] for a
        prefill and [B, 1, Hq, D] for a decode step (the overlay's shapes)."""
        context = get_context()
        if self.k_cache.numel() and self.v_cache.numel():
            store_kvcache(k, v, self.k_cache, self.v_cache, context.slot_mapping)
        if context.is_prefill:
            return self._prefill(q, k, v, context)
        if self.decode_backend == "flash_attn":
            raise NotImplementedError("flash-attn decode is not available on this GPU; "
                                      "configure_model with a custom decode_backend")
        return paged_decode(q, self.k_cache, self.v_cache, context.block_tables,
                            context.context_lens, resources=self.decode_resources,
                            backend=self.decode_backend, scale=self.scale).unsqueeze(1)

    def _prefill(self, q, k, v, context):
        cu_q = context.cu_seqlens_q.tolist()
        cu_k = context.cu_seqlens_k.tolist()
        group = self.num_heads // self.num_kv_heads
        out = torch.empty_like(q)
        for i in range(len(cu_q) - 1):
            nq, nk = cu_q[i + 1] - cu_q[i], cu_k[i + 1] - cu_k[i]
            if context.block_tables is None:
                keys, vals = k[cu_k[i]:cu_k[i + 1]], v[cu_k[i]:cu_k[i + 1]]
            else:  # prefix cache: the whole context is in the paged cache already
                pos = torch.arange(nk, device=q.device)
                blocks = context.block_tables[i, pos // self.k_cache.shape[1]].long()
                keys = self.k_cache[blocks, pos % self.k_cache.shape[1]]
                vals = self.v_cache[blocks, pos % self.k_cache.shape[1]]
            qf = q[cu_q[i]:cu_q[i + 1]].float().transpose(0, 1)                   # [Hq, nq, D]
            kf = keys.float().repeat_interleave(group, dim=1).transpose(0, 1)     # [Hq, nk, D]
            vf = vals.float().repeat_interleave(group, dim=1).transpose(0, 1)
            scores = torch.matmul(qf, kf.transpose(1, 2).contiguous()) * self.scale
            qpos = torch.arange(nk - nq, nk, device=q.device)[:, None]
            scores.masked_fill_(torch.arange(nk, device=q.device)[None, :] > qpos, float("-inf"))
            out[cu_q[i]:cu_q[i + 1]] = torch.matmul(scores.softmax(-1), vf).transpose(0, 1).to(q.dtype)
        return out
