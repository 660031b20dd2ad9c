"""KV-cache writes into 256-slot pages: the step before the decode path.

``store_kvcache`` keeps the signature and checks of the nano-vLLM overlay's
function (overlays/nano-vllm/nanovllm/layers/attention.py:31-38);
``write_pages`` is the page scatter of PagedHybridCache.update
(src/paged_decode/hybrid.py:63-72).  Both run the HIP kernels of
libpaged_decode.so on the current stream, allocate nothing and read no device
memory on the host, so they can be captured in a hipGraph.
"""
import torch

from . import _native


def _require(condition, message):
    if not condition:
        raise ValueError(message)


def store_kvcache(key, value, k_cache, v_cache, slot_mapping):
    """k_cache.view(-1, Hkv*D)[slot_mapping[i]] = key[i] (and V); slot -1 skips.

    key/value: [N, Hkv, D] bf16 with stride(-1) == 1 and stride(1) == D;
    caches: [blocks, block_size, Hkv, D] bf16 with stride(1) == Hkv*D;
    slot_mapping: int32 [N] on the same device.
    """
    _require(key.dim() == 3 and value.shape == key.shape, "key/value must be [N, kv_heads, head_dim]")
    n, hkv, d = key.shape
    _require(key.stride(-1) == 1 and value.stride(-1) == 1, "key/value last dim must be contiguous")
    _require(key.stride(1) == d and value.stride(1) == d, "key/value heads must be contiguous")
    _require(k_cache.stride(1) == hkv * d and v_cache.stride(1) == hkv * d,
             "cache slots must be contiguous rows of kv_heads * head_dim")
    _require(slot_mapping.numel() == n and slot_mapping.dtype == torch.int32,
             "slot_mapping must be int32 with one entry per token")
    _require(key.dtype == torch.bfloat16 and k_cache.dtype == torch.bfloat16 and
             value.dtype == torch.bfloat16 and v_cache.dtype == torch.bfloat16,
             "BF16 key/value and caches required")
    _require(key.is_cuda and all(t.device == key.device
                                 for t in (value, k_cache, v_cache, slot_mapping)),
             "all tensors must be on one CUDA device")
    _native.store_kv(key, value, k_cache, v_cache, slot_mapping)


def write_pages(key, value, k_pages, v_pages, tables, positions):
    """Scatter key/value [B, Hkv, S, D] to pages[table[b, pos // 256], pos % 256].

    ``positions`` is the int64 cache_position vector [S] shared by the batch, as
    in PagedHybridCache.update; pages are [P, 256, Hkv, D] bf16.
    """
    _require(key.dim() == 4 and value.shape == key.shape, "key/value must be [B, kv_heads, S, head_dim]")
    b, hkv, steps, d = key.shape
    _require(k_pages.dim() == 4 and k_pages.shape[1:] == (256, hkv, d) and v_pages.shape == k_pages.shape,
             "pages must be [num_pages, 256, kv_heads, head_dim]")
    _require(k_pages.is_contiguous() and v_pages.is_contiguous(), "pages must be contiguous")
    _require(key.stride(-1) == 1 and value.stride(-1) == 1, "key/value last dim must be contiguous")
    _require(tables.dim() == 2 and tables.shape[0] == b and tables.dtype == torch.int32
             and tables.stride(1) == 1, "tables must be int32 [B, width] with contiguous rows")
    _require(positions.dim() == 1 and positions.numel() == steps and positions.dtype == torch.int64,
             "positions must be int64 [S]")
    _require(key.dtype == torch.bfloat16 and value.dtype == torch.bfloat16 and
             k_pages.dtype == torch.bfloat16 and v_pages.dtype == torch.bfloat16,
             "BF16 key/value and pages required")
    _require(key.is_cuda and all(t.device == key.device
                                 for t in (value, k_pages, v_pages, tables, positions)),
             "key, value, pages, tables and positions must be on one CUDA device")
    _native.store_kv_pages(key, value, k_pages, v_pages, tables, positions)
