"""Random-init Qwen3.5-geometry decoder running the paged decode path end to end.

Mirrors the reference's hybrid runner (src/paged_decode/hybrid.py): the
full-attention layers keep their KV in 256-slot NHD pages written by the HIP
KV-write kernel and decode through ``matched_decode`` / ``paged_decode``;
the linear-attention (Gated DeltaNet) layers run the installed transformers
blocks on their PyTorch path.  The decode step (all layers and the lm_head)
can be captured in one hipGraph and replayed per token.

Differences from the reference, all outside the decode path:
* weights are random (normal, std ``initializer_range``) from a config, not
  loaded from a checkpoint;
* prefill attention is a float32 PyTorch implementation instead of
  flash-attn (not available for this GPU);
* the cache object follows the transformers 5.15 cache interface
  (``update(key, value, layer_idx)``, per-layer linear-attention states);
  the current positions are set on the cache by the runner before each
  forward, as ``cache_position`` was passed in the reference's version.
"""
import torch
from transformers import AttentionInterface
from transformers.cache_utils import LinearAttentionLayer
from transformers.models.qwen3_5 import Qwen3_5ForCausalLM, Qwen3_5TextConfig

from .kv_write import write_pages
from .matched_splitkv import allocate_matched_resources, matched_decode
from .runtime import allocate_resources, paged_decode
from .spec import DecodeSpec

BACKENDS = ("hip_matched", "hip_base", "hip_splitk", "torch")
MODES = ("eager", "graph")


def decoder_config(**overrides):
    """Text config of the end-to-end workload: 24 layers, hidden 2048, full
    attention Hq 8 / Hkv 2 / D 256 every fourth layer, vocab 151936."""
    layers = overrides.pop("num_hidden_layers", 24)
    values = dict(hidden_size=2048, intermediate_size=6144, num_hidden_layers=layers,
                  num_attention_heads=8, num_key_value_heads=2, head_dim=256,
                  vocab_size=151936, linear_num_key_heads=16, linear_key_head_dim=128,
                  linear_num_value_heads=16, linear_value_head_dim=128,
                  linear_conv_kernel_dim=4, initializer_range=0.02,
                  max_position_embeddings=32768,
                  layer_types=["full_attention" if (i + 1) % 4 == 0 else "linear_attention"
                               for i in range(layers)])
    values.update(overrides)
    return Qwen3_5TextConfig(**values)


def random_init_model(config, device="cuda", seed=0):
    """bf16 Qwen3_5ForCausalLM with the transformers initializers, built on `device`."""
    torch.manual_seed(seed)
    with torch.device(device):
        model = Qwen3_5ForCausalLM(config)
    return model.to(torch.bfloat16).eval().requires_grad_(False)


def validate_hybrid_options(backend, mode, batch, max_context):
    if backend not in BACKENDS:
        raise ValueError(f"unknown hybrid backend {backend!r}; expected one of {BACKENDS}")
    if mode not in MODES:
        raise ValueError(f"unknown mode {mode!r}; expected one of {MODES}")
    if mode == "graph" and backend == "torch":
        raise ValueError("the torch reference backend reads lengths on the host; use eager mode")
    if not isinstance(batch, int) or batch < 1:
        raise ValueError("batch must be a positive int")
    if not isinstance(max_context, int) or max_context < 3:
        raise ValueError("max_context must be an int >= 3")


def allocate_hybrid_resources(spec, device, backend):
    if backend == "torch":
        return None
    if backend == "hip_matched":
        return allocate_matched_resources(spec, device)
    return allocate_resources(spec, device, backend)


class PagedHybridCache:
    """Paged KV pool for the full-attention layers plus per-layer linear-attention
    states (transformers ``LinearAttentionLayer``, updated in place so their
    addresses stay fixed across graph replays)."""

    def __init__(self, config, batch, maximum, device):
        self.batch = batch
        self.maximum = maximum
        self.width = (maximum + 255) // 256
        self.prefilled = False
        self.is_prefill = True
        generator = torch.Generator(device="cpu").manual_seed(2026)
        self.tables = torch.randperm(batch * self.width, generator=generator, device="cpu",
                                     dtype=torch.int64).to(device=device, dtype=torch.int32)
        self.tables = self.tables.view(batch, self.width)
        self.lengths = torch.zeros(batch, device=device, dtype=torch.int32)
        self.positions = torch.zeros(1, device=device, dtype=torch.int64)
        shape = (batch * self.width, 256, config.num_key_value_heads, config.head_dim)
        self.pages = {index: (torch.empty(shape, device=device, dtype=torch.bfloat16),
                              torch.empty(shape, device=device, dtype=torch.bfloat16))
                      for index, kind in enumerate(config.layer_types) if kind == "full_attention"}
        self.layers = [LinearAttentionLayer() if kind == "linear_attention" else None
                       for kind in config.layer_types]

    def __len__(self):
        return len(self.layers)

    # ---- linear-attention layers (transformers cache interface)
    def has_previous_state(self, layer_idx=None, state_idx=None):
        layer = self.layers[layer_idx]
        if state_idx is None:
            return all(layer.has_previous_state.values())
        return layer.has_previous_state[state_idx]

    def update_conv_state(self, conv_states, layer_idx, **kwargs):
        return self.layers[layer_idx].update_conv_state(conv_states, 0, **kwargs)

    def update_recurrent_state(self, recurrent_states, layer_idx, **kwargs):
        return self.layers[layer_idx].update_recurrent_state(recurrent_states, 0)

    # ---- full-attention layers
    def update(self, key, value, layer_idx, cache_kwargs=None):
        """Writes key/value [B, Hkv, S, D] at self.positions into the pages."""
        k, v = self.pages[layer_idx]
        write_pages(key, value, k, v, self.tables, self.positions)
        self.lengths.copy_((self.positions[-1] + 1).to(torch.int32).expand(self.batch))
        # Prefill consumes this chunk directly; decode consumes the paged pool.
        return key, value

    def get_seq_length(self, layer_idx=0):
        return 0

    @torch.inference_mode()
    def reset(self):
        self.prefilled = False
        self.is_prefill = True
        self.lengths.zero_()
        for layer in self.layers:
            if layer is not None:
                layer.reset()


def _prefill_attention(query, key, value, scaling):
    """Causal GQA attention in float32 with contiguous operands: [B, S, Hq, D] bf16."""
    b, hq, s, d = query.shape
    group = hq // key.shape[1]
    q = query.float()
    k = key.float().repeat_interleave(group, dim=1)
    v = value.float().repeat_interleave(group, dim=1).contiguous()
    scores = torch.matmul(q, k.transpose(-1, -2).contiguous()) * scaling
    causal = torch.ones(s, s, dtype=torch.bool, device=query.device).triu(1)
    probs = scores.masked_fill(causal, float("-inf")).softmax(-1)
    return torch.matmul(probs, v).transpose(1, 2).to(query.dtype)


def _dense_decode(q, k_pages, v_pages, tables, lengths, scaling):
    """float32 reference decode over the gathered pages (reads lengths on the host)."""
    out = torch.zeros_like(q)
    group = q.shape[1] // k_pages.shape[2]
    for b, length in enumerate(lengths.tolist()):
        if length == 0:
            continue
        pos = torch.arange(length, device=q.device)
        slots = tables[b, pos // 256].long() * 256 + pos % 256
        k = k_pages.view(-1, *k_pages.shape[2:])[slots].float().repeat_interleave(group, dim=1)
        v = v_pages.view(-1, *v_pages.shape[2:])[slots].float().repeat_interleave(group, dim=1)
        scores = torch.einsum("hd,thd->ht", q[b].float(), k) * scaling
        out[b] = torch.einsum("ht,thd->hd", scores.softmax(-1), v).to(q.dtype)
    return out


def _attention(module, query, key, value, attention_mask, scaling, dropout=0.0, **kwargs):
    if attention_mask is not None or dropout:
        raise ValueError("the hybrid runner supports unpadded inference batches only")
    session = module.paged_decode_session
    cache = session.cache
    if cache.is_prefill:
        return _prefill_attention(query, key, value, scaling), None
    q = query.squeeze(2)
    k, v = cache.pages[module.layer_idx]
    if session.backend == "hip_matched":
        output = matched_decode(q, k, v, cache.tables, cache.lengths, resources=session.resources,
                                scale=scaling)
    elif session.backend == "torch":
        output = _dense_decode(q, k, v, cache.tables, cache.lengths, scaling)
    else:
        output = paged_decode(q, k, v, cache.tables, cache.lengths, resources=session.resources,
                              backend=session.backend, scale=scaling)
    return output.unsqueeze(1), None


AttentionInterface.register("paged_decode_lab_hip", _attention)


class HybridRunner:
    """Fixed-batch greedy generation (hybrid.py:106-228 of the reference)."""

    def __init__(self, config=None, *, model=None, backend="hip_matched", mode="eager", batch=1,
                 max_context=2048, device="cuda", seed=0):
        validate_hybrid_options(backend, mode, batch, max_context)
        self.backend, self.mode, self.batch = backend, mode, batch
        self.device = torch.device(device)
        if self.device.type != "cuda":
            raise ValueError("the hybrid runner requires a GPU device")
        self.max_context = max_context
        self.model = model if model is not None else random_init_model(
            config if config is not None else decoder_config(), self.device, seed)
        self.text = self.model.model
        config = self.text.config
        self.spec = DecodeSpec(batch, config.num_attention_heads, config.num_key_value_heads,
                               config.head_dim, max_context)
        self.cache = PagedHybridCache(config, batch, max_context, self.device)
        self.resources = allocate_hybrid_resources(self.spec, self.device, backend)
        for layer in self.text.layers:
            if layer.block_type == "full_attention":
                layer.self_attn.paged_decode_session = self
                layer.self_attn.config._attn_implementation = "paged_decode_lab_hip"
        self.graph = None
        if mode == "graph":
            self._capture()

    @torch.inference_mode()
    def _forward(self, tokens, positions):
        with torch.device(self.device):
            hidden = self.text.embed_tokens(tokens)
            self.cache.positions = positions
            position_ids = positions.view(1, 1, -1).expand(3, self.batch, -1)
            embeddings = self.text.rotary_emb(hidden, position_ids)
            for layer in self.text.layers:
                hidden = layer(hidden, position_embeddings=embeddings, attention_mask=None,
                               past_key_values=self.cache, use_cache=True)
            return self.model.lm_head(self.text.norm(hidden)[:, -1])

    @torch.inference_mode()
    def _capture(self):
        self.cache.reset()
        self._forward(torch.ones(self.batch, 2, dtype=torch.long, device=self.device),
                      torch.arange(2, device=self.device))
        self.cache.prefilled = True
        self.cache.is_prefill = False
        self.graph_tokens = torch.ones(self.batch, 1, dtype=torch.long, device=self.device)
        self.graph_position = torch.tensor([2], dtype=torch.long, device=self.device)
        stream = torch.cuda.Stream(device=self.device)
        stream.wait_stream(torch.cuda.current_stream(self.device))
        with torch.cuda.stream(stream):
            for _ in range(3):
                self._forward(self.graph_tokens, self.graph_position)
        torch.cuda.current_stream(self.device).wait_stream(stream)
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph):
            self.graph_logits = self._forward(self.graph_tokens, self.graph_position)
        self.cache.reset()

    @torch.inference_mode()
    def generate(self, prompts, output_tokens=32, *, observe=False, timing=False):
        """Greedy decoding of `output_tokens` tokens after equally long prompts."""
        if len(prompts) != self.batch or len({len(p) for p in prompts}) != 1:
            raise ValueError("fixed batch requires equally sized, unpadded token sequences")
        length = len(prompts[0])
        if length < 1 or output_tokens < 1 or length + output_tokens > self.max_context:
            raise ValueError("empty input/output or context capacity exceeded")
        self.cache.reset()
        inputs = torch.tensor(prompts, device=self.device, dtype=torch.long)
        logits = self._forward(inputs, torch.arange(length, device=self.device))
        self.cache.prefilled = True
        self.cache.is_prefill = False
        history, saved, intervals = [], [], []
        token = None
        for step in range(output_tokens):
            if step:
                start = end = None
                if timing:
                    start, end = (torch.cuda.Event(enable_timing=True),
                                  torch.cuda.Event(enable_timing=True))
                    start.record()
                if self.graph is None:
                    logits = self._forward(token[:, None],
                                           torch.tensor([length + step - 1], device=self.device))
                else:
                    self.graph_tokens.copy_(token[:, None])
                    self.graph_position.fill_(length + step - 1)
                    self.graph.replay()
                    logits = self.graph_logits
                if timing:
                    end.record()
                    intervals.append((start, end))
            if observe:
                saved.append(logits.detach().float().cpu().clone())
            token = logits.argmax(-1)
            history.append(token.clone())
        torch.cuda.synchronize(self.device)
        return {"token_ids": torch.stack(history, 1).cpu().tolist(), "logits": saved,
                "decode_ms": [a.elapsed_time(b) for a, b in intervals]}
