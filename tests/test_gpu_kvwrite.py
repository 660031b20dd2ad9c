"""GPU parity of the KV-cache write kernels (pd_store_kv, pd_store_kv_pages).

Byte copies, so the gate is bit-exact against oracle/kvwrite.py; untouched
slots keep a NaN poison pattern.
"""
import numpy as np
import pytest
import torch

if not torch.cuda.is_available():
    pytest.skip("needs an MI355X GPU", allow_module_level=True)

from oracle import kvwrite as KW
from paged_decode.kv_write import store_kvcache, write_pages

pytestmark = pytest.mark.gpu
POISON = 0x7FC1  # a bf16 NaN bit pattern


def bits(t):
    return t.view(torch.int16).cpu().numpy()


def rand_bf16(shape, gen):
    return torch.randn(shape, generator=gen, device="cuda").to(torch.bfloat16)


def poisoned(shape):
    return torch.full(shape, POISON, dtype=torch.int16, device="cuda").view(torch.bfloat16)


@pytest.mark.parametrize("hkv,d", [(2, 128), (8, 128), (2, 256), (4, 64)])
def test_store_kvcache_slots_and_padding(hkv, d):
    gen = torch.Generator(device="cuda").manual_seed(hkv * d)
    n, blocks = 37, 4
    # key/value as column slices of a fused qkv row, like the model's split.
    qkv = rand_bf16((n, (8 + 2 * hkv) * d), gen)
    key = qkv[:, 8 * d:(8 + hkv) * d].view(n, hkv, d)
    value = qkv[:, (8 + hkv) * d:].view(n, hkv, d)
    rng = np.random.default_rng(hkv + d)
    slots = rng.permutation(blocks * 256)[:n].astype(np.int32)
    slots[[0, 7, 36]] = -1
    k_cache, v_cache = poisoned((blocks, 256, hkv, d)), poisoned((blocks, 256, hkv, d))
    expected_k, expected_v = bits(k_cache), bits(v_cache)
    store_kvcache(key, value, k_cache, v_cache, torch.from_numpy(slots).cuda())
    torch.cuda.synchronize()
    KW.store_kvcache(bits(key), bits(value), expected_k, expected_v, slots)
    assert (bits(k_cache) == expected_k).all() and (bits(v_cache) == expected_v).all()


@pytest.mark.parametrize("b,hkv,steps,d,start", [(3, 2, 300, 256, 200), (1, 2, 1, 256, 511),
                                                (2, 8, 129, 128, 0), (4, 1, 17, 64, 255)])
def test_write_pages_matches_index_copy(b, hkv, steps, d, start):
    gen = torch.Generator(device="cuda").manual_seed(steps)
    width = (start + steps + 255) // 256 + 1
    tables = torch.from_numpy(np.random.default_rng(steps).permutation(b * width)
                              .reshape(b, width).astype(np.int32)).cuda()
    # [B, S, Hkv, D] projections transposed to [B, Hkv, S, D], as in the model.
    key = rand_bf16((b, steps, hkv, d), gen).transpose(1, 2)
    value = rand_bf16((b, steps, hkv, d), gen).transpose(1, 2)
    positions = torch.arange(start, start + steps, device="cuda", dtype=torch.int64)
    k_pages, v_pages = poisoned((b * width, 256, hkv, d)), poisoned((b * width, 256, hkv, d))
    ek, ev = bits(k_pages), bits(v_pages)
    write_pages(key, value, k_pages, v_pages, tables, positions)
    torch.cuda.synchronize()
    KW.write_pages(bits(key.contiguous()), bits(value.contiguous()), ek, ev, tables.cpu().numpy(),
                   positions.cpu().numpy())
    assert (bits(k_pages) == ek).all() and (bits(v_pages) == ev).all()


def test_write_pages_graph_replay_with_new_positions():
    gen = torch.Generator(device="cuda").manual_seed(5)
    b, hkv, d, width = 2, 2, 256, 4
    tables = torch.tensor([[5, 1, 7, 3], [0, 6, 2, 4]], dtype=torch.int32, device="cuda")
    key = rand_bf16((b, hkv, 1, d), gen)
    value = rand_bf16((b, hkv, 1, d), gen)
    position = torch.zeros(1, dtype=torch.int64, device="cuda")
    k_pages, v_pages = poisoned((8, 256, hkv, d)), poisoned((8, 256, hkv, d))
    ek, ev = bits(k_pages), bits(v_pages)
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        write_pages(key, value, k_pages, v_pages, tables, position)
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    KW.write_pages(bits(key), bits(value), ek, ev, tables.cpu().numpy(), np.array([0]))
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        write_pages(key, value, k_pages, v_pages, tables, position)
    for pos in (255, 256, 700):
        position.fill_(pos)
        key.copy_(rand_bf16(key.shape, gen))
        value.copy_(rand_bf16(value.shape, gen))
        graph.replay()
        torch.cuda.synchronize()
        KW.write_pages(bits(key), bits(value), ek, ev, tables.cpu().numpy(), np.array([pos]))
        assert (bits(k_pages) == ek).all() and (bits(v_pages) == ev).all(), pos


def test_contract_errors():
    n, hkv, d = 4, 2, 128
    key = torch.zeros(n, hkv, d, dtype=torch.bfloat16, device="cuda")
    cache = torch.zeros(2, 256, hkv, d, dtype=torch.bfloat16, device="cuda")
    with pytest.raises(ValueError, match="int32"):
        store_kvcache(key, key, cache, cache, torch.zeros(n, dtype=torch.int64, device="cuda"))
    with pytest.raises(ValueError, match="contiguous"):
        store_kvcache(key.transpose(1, 2).contiguous().transpose(1, 2), key, cache, cache,
                      torch.zeros(n, dtype=torch.int32, device="cuda"))
    with pytest.raises(ValueError, match="BF16"):
        store_kvcache(key.float(), key.float(), cache, cache, torch.zeros(n, dtype=torch.int32, device="cuda"))
    key4 = torch.zeros(1, hkv, 3, 96, dtype=torch.bfloat16, device="cuda")
    pages = torch.zeros(2, 256, hkv, 96, dtype=torch.bfloat16, device="cuda")
    with pytest.raises(ValueError, match="head_dim"):
        write_pages(key4, key4, pages, pages, torch.zeros(1, 2, dtype=torch.int32, device="cuda"),
                    torch.arange(3, device="cuda"))
