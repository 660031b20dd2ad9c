"""Capacity-aligned split-KV with normalized FP32 partials + LSE.

Mirrors matched_splitkv.py of the reference (src/paged_decode/matched_splitkv.py:15-150):
``MatchedResources``, ``allocate_matched_resources`` and ``matched_decode``,
with the same plan, workspace shapes, contract checks and error messages.

By default ``matched_decode`` launches the partition and the LSE merge as two
kernels (pd_partition, pd_lse_merge), like the reference.  Resources
allocated with ``fused=True`` carry a zeroed int32 counter per (sequence, kv
head) and run both in one launch instead (pd_matched_decode: the last
workgroup of each GQA group merges it).  Both give bit-identical outputs; the
two-launch path is faster on MI355X at the benchmark shapes, because the
single launch exchanges the partials between XCDs through device-coherent
memory inside the kernel.
"""
from dataclasses import dataclass
import math

import torch

from . import _native
from .runtime import _validate
from .splitkv_plan import make_splitkv_plan

# int32 split counters per (sequence, kv head) of the fused launch
# (PD_FUSED_COUNTERS_PER_GROUP): one per wavefront column slice of the
# single-tile kernel, each on a 128-byte line of its own (the multi-tile
# kernels use the first).
COUNTERS_PER_GROUP = 128


@dataclass
class MatchedResources:
    spec: object
    plan: object
    out: torch.Tensor
    partials: torch.Tensor
    lse: torch.Tensor
    counters: torch.Tensor | None = None


def allocate_matched_resources(spec, device, *, num_splits=0, fused=False):
    device = torch.device(device)
    if device.type != "cuda":
        raise ValueError("matched resources require CUDA")
    plan = make_splitkv_plan(spec, torch.cuda.get_device_properties(device).multi_processor_count,
                             num_splits=num_splits)
    shape = (spec.max_batch, spec.num_heads, plan.splits)
    return MatchedResources(
        spec, plan,
        torch.empty((spec.max_batch, spec.num_heads, spec.head_dim), device=device,
                    dtype=torch.bfloat16),
        torch.empty((*shape, spec.head_dim), device=device, dtype=torch.float32),
        torch.empty(shape, device=device, dtype=torch.float32),
        torch.zeros((spec.max_batch * spec.num_kv_heads * COUNTERS_PER_GROUP,), device=device,
                    dtype=torch.int32)
        if fused else None)


def _check_matched(q, tables, resources, scale):
    if scale <= 0 or not math.isfinite(scale):
        raise ValueError("positive finite scale required")
    spec, plan = resources.spec, resources.plan
    if q.shape[0] != spec.max_batch or tables.shape[1] != spec.table_width:
        raise ValueError("matched plan requires its fixed batch and table capacity")
    shape = (spec.max_batch, spec.num_heads, plan.splits)
    for tensor, geometry in ((resources.lse, shape),
                             (resources.partials, (*shape, spec.head_dim))):
        if (tensor.shape != geometry or tensor.get_device() != q.get_device()
                or tensor.dtype != torch.float32 or not tensor.is_contiguous()):
            raise ValueError("invalid matched workspace")
    counters = resources.counters
    if counters is not None and (
            counters.shape != (spec.max_batch * spec.num_kv_heads * COUNTERS_PER_GROUP,)
            or counters.get_device() != q.get_device()
            or counters.dtype != torch.int32 or not counters.is_contiguous()):
        raise ValueError("invalid matched workspace")


def matched_decode(q, k, v, tables, lengths, *, resources, scale=None):
    """Return the borrowed [max_batch, Hq, D] bf16 output (overwritten by the next call)."""
    scale = q.shape[-1] ** -.5 if scale is None else float(scale)
    _validate(q, k, v, tables, lengths, resources, "hip_base", scale)
    _check_matched(q, tables, resources, scale)
    spec, plan = resources.spec, resources.plan
    # With counters the fused launch; without, the partition then the LSE merge
    # (matched_splitkv.py:147-149), or the partition alone for a plan of one split of
    # several tiles, whose merge is the identity (the same bits).
    _native.matched_decode(q, k, v, tables, lengths, resources.partials, resources.lse,
                           resources.counters, resources.out, spec.num_kv_heads, plan.splits,
                           plan.tokens_per_split, plan.tile_tokens, scale)
    return resources.out
