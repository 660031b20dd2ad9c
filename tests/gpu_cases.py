"""GPU-side helpers for the parity tests (torch tensors on the MI355X)."""
import numpy as np
import torch

from parity import assert_parity, record


def to_gpu(case, device="cuda"):
    q, k, v, table, lengths = case
    bf = lambda x: torch.from_numpy(np.ascontiguousarray(x)).to(device).to(torch.bfloat16)
    return (bf(q), bf(k), bf(v), torch.from_numpy(np.ascontiguousarray(table)).to(device),
            torch.from_numpy(np.ascontiguousarray(lengths)).to(device))


def to_np(t):
    return t.detach().float().cpu().numpy()


def poison(*tensors):
    """Fills float tensors with NaN (the reference's check that a launch writes what it
    should, tools/resident_experiment.py:117-121): a slot a kernel should have written but
    did not then shows as NaN in the output or the workspace."""
    for t in tensors:
        if t is not None:
            t.fill_(float("nan"))


WORKSPACE_FIELDS = ("out", "partials", "lse", "maxima", "denoms", "accums", "chunk_maxima",
                    "chunk_denoms", "chunk_accums")


def poison_workspace(res):
    """NaN into the output and every float workspace of paged_decode or matched_decode
    resources (never the fused counters, which must stay zero between calls)."""
    poison(*(getattr(res, name, None) for name in WORKSPACE_FIELDS))


def assert_within_one_ulp(actual, expected, where="", ambiguity=None, ambiguous_p=None):
    """Parity gate of tests/parity.py (one bf16 ulp beyond the oracle's rounding-ambiguity
    bound, at most 0.5% of outputs beyond one ulp); ``ambiguous_p`` [B, Hq], the oracle's
    count of ambiguous p values per row, goes into the record of the worst output."""
    actual = to_np(actual) if isinstance(actual, torch.Tensor) else actual
    return assert_parity(actual, expected, where, ambiguity, ambiguous_p)["one_ulp"]


def torch_dense(q, k, v, tables, lengths, scale=None):
    """FP32 gather + dense softmax on the device (restates torch_reference.py:5-17)."""
    result = torch.zeros_like(q, dtype=torch.float32)
    group = q.shape[1] // k.shape[2]
    scale = q.shape[-1] ** -0.5 if scale is None else scale
    for b, length in enumerate(lengths.cpu().tolist()):
        if length == 0:
            continue
        pos = torch.arange(length, device=q.device)
        pages = tables[b, pos // 256].long()
        keys = k[pages, pos % 256].float().repeat_interleave(group, dim=1)   # [n, Hq, D]
        vals = v[pages, pos % 256].float().repeat_interleave(group, dim=1)
        scores = torch.matmul(keys.permute(1, 0, 2).contiguous(),
                              q[b].float().unsqueeze(-1)).squeeze(-1) * scale  # [Hq, n]
        probs = scores.softmax(-1)
        result[b] = torch.matmul(probs.unsqueeze(1), vals.permute(1, 0, 2).contiguous()).squeeze(1)
    return result


def assert_close_dense(actual, expected, where=""):
    """The reference's dense gate (2e-2, tests/test_gpu.py:44-48); max-abs and RMSE are
    recorded for the run's parity summary."""
    assert torch.isfinite(actual).all()
    torch.testing.assert_close(actual.float(), expected.float(), atol=2e-2, rtol=2e-2)
    diff = actual.float() - expected.float()
    record(where, max_abs_vs_dense=float(diff.abs().max()) if diff.numel() else 0.0,
           rmse_vs_dense=float(diff.square().mean().sqrt()) if diff.numel() else 0.0)


def pooled_case(lengths, hq, hkv, dim, capacity, pool_pages, seed, device="cuda"):
    """Device inputs at full benchmark size: each sequence's pages are drawn without
    replacement from a pool of ``pool_pages`` physical pages per cache, in random
    order.  Only live pages get N(0, 1) bf16 values; the rest of the pool holds NaN, so
    a read outside the live tokens poisons the output.  Table entries past a row's live
    pages are -1."""
    gen = torch.Generator(device=device).manual_seed(seed)
    width = (capacity + 255) // 256
    live = [(int(n) + 255) // 256 for n in lengths]
    physical = torch.randperm(pool_pages, device=device, generator=gen)[: sum(live)]
    table = torch.full((len(lengths), width), -1, dtype=torch.int32, device=device)
    offset = 0
    for b, n in enumerate(live):
        table[b, :n] = physical[offset:offset + n].to(torch.int32)
        offset += n
    k = torch.full((pool_pages, 256, hkv, dim), float("nan"), dtype=torch.bfloat16, device=device)
    v = torch.full_like(k, float("nan"))
    for chunk in torch.split(physical.long(), 512):
        k[chunk] = torch.randn((len(chunk), 256, hkv, dim), generator=gen, device=device,
                               dtype=torch.bfloat16)
        v[chunk] = torch.randn((len(chunk), 256, hkv, dim), generator=gen, device=device,
                               dtype=torch.bfloat16)
    q = torch.randn((len(lengths), hq, dim), generator=gen, device=device, dtype=torch.bfloat16)
    lens = torch.tensor([int(n) for n in lengths], dtype=torch.int32, device=device)
    return q, k, v, table, lens


def host_rows(q, k, v, table, lengths, rows):
    """The sequences ``rows`` of a device case as a compact NumPy case for the oracle:
    their live pages copied to the host and renumbered, the table -1 padded."""
    lens = lengths[rows].cpu().numpy().astype(np.int32)
    live = [(int(n) + 255) // 256 for n in lens]
    pages = torch.cat([table[r, :n] for r, n in zip(rows, live)]).long()
    compact = np.full((len(rows), table.shape[1]), -1, dtype=np.int32)
    offset = 0
    for i, n in enumerate(live):
        compact[i, :n] = np.arange(offset, offset + n)
        offset += n
    return (to_np(q[rows]), to_np(k[pages]), to_np(v[pages]), compact, lens)
