"""GPU-side helpers for the parity tests (torch tensors on the MI355X)."""
import numpy as np
import torch

from parity import assert_parity


def to_gpu(case, device="cuda"):
    q, k, v, table, lengths = case
    bf = lambda x: torch.from_numpy(np.ascontiguousarray(x)).to(device).to(torch.bfloat16)
    return (bf(q), bf(k), bf(v), torch.from_numpy(np.ascontiguousarray(table)).to(device),
            torch.from_numpy(np.ascontiguousarray(lengths)).to(device))


def to_np(t):
    return t.detach().float().cpu().numpy()


def assert_within_one_ulp(actual, expected, where="", ambiguity=None):
    """Parity gate of tests/parity.py (one bf16 ulp beyond the oracle's rounding-ambiguity
    bound, at most 1% of outputs beyond one ulp)."""
    actual = to_np(actual) if isinstance(actual, torch.Tensor) else actual
    return assert_parity(actual, expected, where, ambiguity)["one_ulp"]


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


def assert_close_dense(actual, expected):
    assert torch.isfinite(actual).all()
    torch.testing.assert_close(actual.float(), expected.float(), atol=2e-2, rtol=2e-2)
