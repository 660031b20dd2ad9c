"""Engine initialization hook: attach decode resources to a model's attention layers.

Restates ``configure_model`` of the reference (src/paged_decode/integration.py:8-26),
which the nano-vLLM overlay's ModelRunner calls once after allocating the KV cache
(overlays/nano-vllm/nanovllm/engine/model_runner.py:37-38).  No monkeypatching: a
layer opts in by carrying ``k_cache``, ``v_cache``, ``num_heads``, ``num_kv_heads`` and
``head_dim``; the hook sets ``decode_backend`` and ``decode_resources`` on it.

Layers run one after another on one stream and each layer's projection consumes its
borrowed attention output before the next layer runs, so layers of the same geometry
share one Resources object (one output buffer and one split workspace).
"""
import torch

from .runtime import allocate_resources
from .spec import DecodeSpec

_LAYER_ATTRS = ("k_cache", "v_cache", "num_heads", "num_kv_heads", "head_dim")


def configure_model(model, config):
    """Give every attention layer of ``model`` the backend and resources ``config`` asks for.

    ``config`` needs ``decode_backend``, ``max_num_seqs``, ``max_model_len`` and
    ``kvcache_block_size`` (the nano-vLLM Config fields).  ``flash_attn`` leaves the model
    untouched.  Raises ValueError for a non-BF16 KV cache or a model without layers.
    """
    if config.decode_backend == "flash_attn":
        return
    by_geometry = {}
    for layer in model.modules():
        if not all(hasattr(layer, name) for name in _LAYER_ATTRS):
            continue
        if layer.k_cache.dtype != torch.bfloat16:
            raise ValueError("custom nano-vLLM decode requires a BF16 model")
        spec = DecodeSpec(config.max_num_seqs, layer.num_heads, layer.num_kv_heads,
                          layer.head_dim, config.max_model_len, config.kvcache_block_size)
        resources = by_geometry.get(spec)
        if resources is None:
            resources = by_geometry[spec] = allocate_resources(spec, layer.k_cache.device,
                                                               config.decode_backend)
        layer.decode_backend = config.decode_backend
        layer.decode_resources = resources
    if not by_geometry:
        raise ValueError("no compatible attention layers found")
