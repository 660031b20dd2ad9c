"""Host logic of the engine hook (configure_model) and the engine-side decode metadata.

Follows the reference's nano-vLLM integration (src/paged_decode/integration.py:8-26,
overlays/nano-vllm/nanovllm/engine/model_runner.py:130-134,179-195,250-251).  Runs on
the CPU: resources are allocated on the layers' cache device.
"""
from types import SimpleNamespace

import pytest
import torch
from torch import nn

from paged_decode.engine_attention import Attention, decode_metadata, graph_batch_sizes
from paged_decode.integration import configure_model
from paged_decode.spec import DecodeSpec


def _config(backend="hip_splitk", seqs=8, model_len=1000):
    return SimpleNamespace(decode_backend=backend, max_num_seqs=seqs, max_model_len=model_len,
                           kvcache_block_size=256)


def _model(geometries, dtype=torch.bfloat16):
    layers = nn.ModuleList()
    for hq, hkv, d in geometries:
        layer = Attention(hq, d, d ** -0.5, hkv)
        layer.k_cache = torch.zeros((2, 256, hkv, d), dtype=dtype)
        layer.v_cache = torch.zeros_like(layer.k_cache)
        layers.append(layer)
    return nn.Sequential(nn.Linear(2, 2), layers)


def test_layers_of_one_geometry_share_resources():
    model = _model([(16, 8, 128), (16, 8, 128), (32, 4, 64), (16, 8, 128)])
    configure_model(model, _config())
    layers = [m for m in model.modules() if isinstance(m, Attention)]
    assert all(layer.decode_backend == "hip_splitk" for layer in layers)
    assert layers[0].decode_resources is layers[1].decode_resources is layers[3].decode_resources
    assert layers[2].decode_resources is not layers[0].decode_resources
    res = layers[0].decode_resources
    assert res.spec == DecodeSpec(8, 16, 8, 128, 1000)
    assert res.out.shape == (8, 16, 128) and res.out.dtype == torch.bfloat16
    assert res.accums.shape == (8, 16, 1, 128)          # ceil(1000 / 1024) partitions
    assert layers[2].decode_resources.spec == DecodeSpec(8, 32, 4, 64, 1000)


def test_base_backend_allocates_no_split_workspace_and_aliases_are_kept():
    model = _model([(8, 2, 256)])
    configure_model(model, _config("triton_base"))
    layer = next(m for m in model.modules() if isinstance(m, Attention))
    assert layer.decode_backend == "triton_base"
    assert layer.decode_resources.maxima is None and layer.decode_resources.accums is None


def test_flash_attn_leaves_the_model_untouched():
    model = _model([(8, 2, 128)])
    configure_model(model, _config("flash_attn"))
    layer = next(m for m in model.modules() if isinstance(m, Attention))
    assert layer.decode_backend == "flash_attn" and layer.decode_resources is None


def test_non_bf16_cache_and_empty_model_are_rejected():
    with pytest.raises(ValueError, match="BF16 model"):
        configure_model(_model([(8, 2, 128)], dtype=torch.float16), _config())
    with pytest.raises(ValueError, match="no compatible attention layers"):
        configure_model(nn.Sequential(nn.Linear(2, 2)), _config())
    with pytest.raises(ValueError, match="head_dim"):
        configure_model(_model([(8, 2, 96)]), _config())


def test_decode_metadata_slots_lengths_and_padding():
    slots, lens, tables = decode_metadata([[7, 3], [5], [1, 2, 9]], [300, 1, 513], device="cpu")
    # last token of a 300-token sequence: block 3 (second block), offset 43
    assert slots.tolist() == [3 * 256 + 43, 5 * 256 + 0, 9 * 256 + 0]
    assert lens.tolist() == [300, 1, 513]
    assert tables.tolist() == [[7, 3, -1], [5, -1, -1], [1, 2, 9]]
    assert slots.dtype == lens.dtype == tables.dtype == torch.int32


def test_graph_buckets():
    assert graph_batch_sizes(512) == [1, 2, 4, 8] + list(range(16, 513, 16))
    assert graph_batch_sizes(20) == [1, 2, 4, 8, 16, 20]
    assert graph_batch_sizes(3) == [1, 2, 3]
    assert graph_batch_sizes(1000)[-1] == 512


def test_flash_attn_decode_raises_on_this_platform():
    from paged_decode.engine_attention import reset_context
    reset_context()
    layer = Attention(8, 64, 0.125, 2)
    q = torch.zeros((1, 8, 64), dtype=torch.bfloat16)
    k = torch.zeros((1, 2, 64), dtype=torch.bfloat16)
    with pytest.raises(NotImplementedError, match="custom decode_backend"):
        layer(q, k, k)


def test_decode_timings_skip_prefill_and_disabled_steps():
    """Prefill steps and steps with timing off run untimed (no CUDA events needed)."""
    from paged_decode.engine_attention import DecodeTimings
    timings = DecodeTimings(enabled=False)
    assert timings.run(lambda: 7, 4) == 7
    timings.enabled = True
    assert timings.run(lambda: 8, 4, is_prefill=True) == 8
    assert timings.records == [] and timings.intervals() == []
