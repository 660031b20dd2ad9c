"""Host side of the paged_decode backends: argument checks, HIP launches, and the
preallocated output and split workspace they write.

Mirrors runtime.py of the reference (src/paged_decode/runtime.py:15-117):
``Resources``, ``allocate_resources``, ``validate_device_metadata``,
``paged_decode`` and the host-only ``_validate`` contract with the same error
messages.  Kernels are the HIP ones in libpaged_decode.so.

The launches never look at tensor contents: page ids and lengths are taken as
given.  Tables that come from outside a scheduler should be checked once with
validate_device_metadata, which does read them (and synchronizes).  A call
allocates nothing, never synchronizes and never reads device memory on the
host, so it can be captured into a hipGraph (torch.cuda.graph) after the
resources are allocated and replayed with new lengths, pages and KV contents.

Small batches.  hip_base and hip_splitk walk each sequence in one workgroup per
kv head group.  When a batch has fewer such walks than half of the device's
CUs, paged_decode cuts each sequence's table width into chunks
(pd_plan_chunks), runs the fixed-split partition over them (one workgroup per
chunk) into the resources' chunk workspace and merges the chunks into the
output (pd_ml_merge): the same attention with other float32 rounding, within
the one-ulp parity gate of either backend's oracle.  The cut depends on the
batch only through its next power of two and on the capacity, not the live
table width, so the decode graph of a padded batch bucket gives the live rows
the bits of the eager call.  The chunk workspace has no counterpart in the
reference; resources built without it take the walk.
"""
from dataclasses import dataclass, field
import math

import torch

from . import _native
from .spec import DecodeSpec, PARTITION_SIZE, canonical_backend


@dataclass
class Resources:
    spec: DecodeSpec
    out: torch.Tensor
    maxima: torch.Tensor | None = None
    denoms: torch.Tensor | None = None
    accums: torch.Tensor | None = None
    # Small-batch chunk workspace (flat float32: (m, l) per chunk row, D accumulators
    # per row) and the CU count it was sized for; None / 0 when no batch needs it.
    chunk_maxima: torch.Tensor | None = None
    chunk_denoms: torch.Tensor | None = None
    chunk_accums: torch.Tensor | None = None
    sm_count: int = 0
    _chunk_plans: dict = field(default_factory=dict, repr=False, compare=False)
    # Shaped views of the chunk workspace by (batch, chunks), made once per shape.
    _chunk_views: dict = field(default_factory=dict, repr=False, compare=False)


def _device_cus(device):
    return torch.cuda.get_device_properties(torch.device(device)).multi_processor_count


def allocate_resources(spec, device, backend="hip_splitk"):
    try:
        backend = canonical_backend(backend)
    except ValueError:
        raise ValueError("resources require a custom backend") from None
    out = torch.empty((spec.max_batch, spec.num_heads, spec.head_dim),
                      dtype=torch.bfloat16, device=device)
    result = Resources(spec, out)
    if backend == "hip_splitk":
        shape = (spec.max_batch, spec.num_heads, spec.partitions)
        result.maxima = torch.empty(shape, device=device, dtype=torch.float32)
        result.denoms = torch.empty(shape, device=device, dtype=torch.float32)
        result.accums = torch.empty((*shape, spec.head_dim), device=device, dtype=torch.float32)
    if torch.device(device).type == "cuda":
        result.sm_count = _device_cus(device)
        rows = _native.chunk_rows(spec.max_batch, spec.num_heads, spec.num_kv_heads,
                                  spec.head_dim, result.sm_count)
        if rows:
            result.chunk_maxima = torch.empty(rows, device=device, dtype=torch.float32)
            result.chunk_denoms = torch.empty(rows, device=device, dtype=torch.float32)
            result.chunk_accums = torch.empty(rows * spec.head_dim, device=device,
                                              dtype=torch.float32)
    return result


def _chunk_plan(resources, batch, width):
    """(chunks, chunk_tokens) for a call of ``batch`` sequences over a table of ``width``
    pages, or None when the backend runs as it is (a batch that fills the CUs, or resources
    without a chunk workspace large enough).  The cut is planned at the capacity's table
    width and runs the chunks that cover ``width`` pages, so that a sequence gets the
    same bits from the live table as from the capacity-wide one a graph was captured with
    (pd_plan_chunks)."""
    key = (batch, width)
    plans = resources._chunk_plans
    if key not in plans:
        spec, plan = resources.spec, None
        workspace = (resources.chunk_maxima, resources.chunk_denoms, resources.chunk_accums)
        if resources.sm_count > 0 and all(
                t is not None and t.dtype == torch.float32 and t.is_contiguous()
                and t.device == resources.out.device for t in workspace):
            full, tokens = _native.plan_chunks(batch, spec.num_heads, spec.num_kv_heads,
                                               spec.head_dim, spec.table_width,
                                               resources.sm_count)
            chunks = -(-width * 256 // tokens)
            rows = batch * spec.num_heads * chunks
            if (full > 1 and workspace[0].numel() >= rows and workspace[1].numel() >= rows
                    and workspace[2].numel() >= rows * spec.head_dim):
                plan = (chunks, tokens)
        plans[key] = plan
    return plans[key]


def validate_device_metadata(table, lengths, num_pages, max_context_len):
    """Check table and length contents on the host.

    The contents are copied off the device, so this synchronizes: call it once for
    tables from outside a scheduler, never inside graph capture or the decode loop."""
    if torch.cuda.is_available() and torch.cuda.is_current_stream_capturing():
        raise RuntimeError("metadata content validation cannot run during graph capture")
    if table.dim() != 2 or lengths.dim() != 1 or table.shape[0] != lengths.shape[0]:
        raise ValueError("metadata batch dimensions differ")
    # reference.py:14-15: integral dtypes only (no float truncation, no bool).
    for x in (table, lengths):
        if x.dtype.is_floating_point or x.dtype.is_complex or x.dtype == torch.bool:
            raise ValueError("metadata must be integral")
    _native.validate_metadata(_host_int32(table), _host_int32(lengths), int(num_pages),
                              int(max_context_len))


def _host_int32(x):
    """Host int32 copy; wider values saturate to [-1, 2^31 - 1] instead of wrapping, so a
    negative or out-of-range length or live page entry is still rejected after narrowing."""
    x = x.detach().to("cpu")
    if x.dtype != torch.int32:
        x = x.to(torch.int64).clamp(-1, 2 ** 31 - 1).to(torch.int32)
    return x.contiguous()


def _aligned(t):
    return t.data_ptr() % 16 == 0


def _validate(q, k, v, tables, lengths, resources, backend, scale):
    if backend not in ("hip_base", "hip_splitk"):
        raise ValueError("unknown custom backend")
    spec = resources.spec
    # get_device() is the CUDA index, -1 on the CPU (no torch.device objects built).
    device = q.get_device()
    if device < 0 or not (k.get_device() == v.get_device() == tables.get_device()
                          == lengths.get_device() == resources.out.get_device() == device):
        raise ValueError("all tensors must be on the same CUDA device")
    if q.dtype != torch.bfloat16 or k.dtype != q.dtype or v.dtype != q.dtype:
        raise ValueError("custom decode supports BF16 Q/K/V only")
    if q.ndim != 3 or q.shape[1:] != (spec.num_heads, spec.head_dim):
        raise ValueError("Q must have shape [batch, query_heads, head_dim]")
    batch = q.shape[0]
    if not 0 < batch <= spec.max_batch or q.stride(-1) != 1:
        raise ValueError("Q batch exceeds capacity or innermost dimension is not contiguous")
    if q.stride(0) % 8 or q.stride(1) % 8 or not _aligned(q):
        raise ValueError("Q rows must be 16-byte aligned (strides multiples of 8 elements)")
    if k.ndim != 4 or k.shape[1:] != (256, spec.num_kv_heads, spec.head_dim):
        raise ValueError("KV must use NHD pages [pages,256,kv_heads,head_dim]")
    if k.shape != v.shape or not k.is_contiguous() or not v.is_contiguous() or k.shape[0] == 0:
        raise ValueError("K/V must have matching nonempty contiguous storage")
    if not (_aligned(k) and _aligned(v)):
        raise ValueError("K/V storage must be 16-byte aligned")
    if tables.ndim != 2 or tables.shape[0] != batch or tables.stride(1) != 1:
        raise ValueError("block table must have shape [batch,capacity] and contiguous rows")
    # An eager caller may pass a table narrower than the capacity (its live pages only).
    if not 0 < tables.shape[1] <= spec.table_width:
        raise ValueError("block table width outside configured capacity")
    if lengths.shape != (batch,) or not lengths.is_contiguous():
        raise ValueError("context lengths must be a contiguous [batch] tensor")
    if tables.dtype != torch.int32 or lengths.dtype != torch.int32:
        raise ValueError("block tables and context lengths must be int32")
    if not math.isfinite(scale):
        raise ValueError("scale must be finite")
    if (resources.out.shape != (spec.max_batch, spec.num_heads, spec.head_dim)
            or resources.out.dtype != q.dtype or not resources.out.is_contiguous()):
        raise ValueError("invalid output buffer")
    if backend == "hip_splitk":
        shape = (spec.max_batch, spec.num_heads, spec.partitions)
        for tensor, expected in ((resources.maxima, shape), (resources.denoms, shape),
                                 (resources.accums, (*shape, spec.head_dim))):
            if (tensor is None or tensor.shape != expected or tensor.get_device() != device
                    or tensor.dtype != torch.float32 or not tensor.is_contiguous()):
                raise ValueError("invalid or missing preallocated split-K workspace")


def paged_decode(q, k, v, tables, lengths, *, resources, backend="hip_base", scale=None):
    """Attention of one query token per sequence; returns ``resources.out[:B]``.

    The returned tensor is a view of the resources' output buffer, so the next call with
    the same resources overwrites it.  The resources may not share memory with the inputs,
    and two streams may not use them at once.  Contract on contents (not checked here):
    every live table entry names a page of K/V, each length lies in [0, max_context_len]
    and needs at most the table's width of pages; entries past a row's live pages may be
    -1.
    """
    scale = q.shape[-1] ** -0.5 if scale is None else float(scale)
    backend = canonical_backend(backend)
    _validate(q, k, v, tables, lengths, resources, backend, scale)
    spec = resources.spec
    b = q.shape[0]
    chunked = _chunk_plan(resources, b, tables.shape[1])
    if chunked is not None:
        chunks, tokens = chunked
        views = resources._chunk_views.get((b, chunks))
        if views is None:
            rows = b * spec.num_heads * chunks
            shape = (b, spec.num_heads, chunks)
            views = (resources.chunk_maxima[:rows].view(shape),
                     resources.chunk_denoms[:rows].view(shape),
                     resources.chunk_accums[:rows * spec.head_dim].view(*shape, spec.head_dim))
            resources._chunk_views[(b, chunks)] = views
        maxima, denoms, accums = views
        _native.split_fixed(q, k, v, tables, lengths, maxima, denoms, accums, spec.num_kv_heads,
                            chunks, tokens, scale)
        _native.ml_merge(maxima, denoms, accums, resources.out, b)
        return resources.out[:b]
    if backend == "hip_base":
        _native.base(q, k, v, tables, lengths, resources.out, spec.num_kv_heads, scale)
    else:
        # _split + _merge (runtime.py:111-116 of the reference) in one call: the walking
        # workgroups merge their partitions themselves when they fill the device.
        _native.split_decode(q, k, v, tables, lengths, resources.maxima, resources.denoms,
                             resources.accums, resources.out, spec.num_kv_heads,
                             spec.partitions, PARTITION_SIZE, scale)
    return resources.out[:b]
