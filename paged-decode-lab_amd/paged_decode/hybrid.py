"""Random-init Qwen3.5-geometry decoder running the paged decode path end to end.

The counterpart of the reference's hybrid runner (src/paged_decode/hybrid.py:15-228):
the full-attention layers keep their KV in 256-slot NHD pages, written by the HIP
KV-write kernel and read by ``matched_decode`` / ``paged_decode``; the
linear-attention (Gated DeltaNet) layers run the installed transformers blocks on
their PyTorch path.  A decode step (every layer and the lm_head) runs eagerly or as
one replayed hipGraph.

Structure:
* ``PagedKVPool``: the K and V pages of every full-attention layer in one device
  block ``[layers, 2, pages, 256, Hkv, D]``, one page table shared by the layers
  (a seeded random physical page order), and the step's device ``positions`` /
  ``lengths``.  The lengths are set once per step, before the layers run.
* ``HybridCache``: the transformers 5.15 cache protocol on top of the pool
  (``update(key, value, layer_idx)`` for full attention, per-layer
  ``LinearAttentionLayer`` states, which transformers keeps at fixed addresses).
* ``DecodeStepGraph``: the decode step captured on first use, after a prefill,
  when every linear-attention state already exists at its final address.  The
  states are saved, the step is warmed up on a side stream, the states are put
  back, and the step is captured; later generations replay the same graph.
* ``HybridRunner.generate``: greedy decoding, optionally teacher-forced
  (``forced=``, hybrid.py:185,221 of the reference), returning the predicted and
  the fed tokens, per-step logits and per-step timings.

Differences from the reference, all outside the decode path: random weights
from a config instead of a checkpoint (no tokenizer, so no decoded text);
float32 PyTorch prefill attention instead of flash-attn (not available for this
GPU); the float32 ``torch`` backend takes the place of the flash-attn decode peer.
"""
import dataclasses

import numpy as np
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
PAGE = 256
TABLE_SEED = 2026


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
    """Option checks of the runner (the reference's hybrid_options.py)."""
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
    """Decode workspace of one backend (none for the float32 torch backend)."""
    if backend == "torch":
        return None
    if backend == "hip_matched":
        return allocate_matched_resources(spec, device)
    return allocate_resources(spec, device, backend)


def seeded_page_table(batch, width, seed=TABLE_SEED):
    """A random physical order of the batch's ``batch * width`` pages, int32 [batch, width]."""
    order = np.random.default_rng(seed).permutation(batch * width).astype(np.int32)
    return torch.from_numpy(order.reshape(batch, width))


class PagedKVPool:
    """KV pages of the full-attention layers, their page table and the step's lengths."""

    def __init__(self, layer_ids, batch, capacity, kv_heads, head_dim, device):
        self.batch = batch
        self.width = -(-capacity // PAGE)
        self.slot = {layer: i for i, layer in enumerate(layer_ids)}
        self.block = torch.empty((len(layer_ids), 2, batch * self.width, PAGE, kv_heads, head_dim),
                                 device=device, dtype=torch.bfloat16)
        self.tables = seeded_page_table(batch, self.width).to(device)
        self.positions = torch.zeros(1, device=device, dtype=torch.int64)
        self.lengths = torch.zeros(batch, device=device, dtype=torch.int32)

    def pages(self, layer_idx):
        """(K, V) pages of one layer, each a contiguous [pages, 256, Hkv, D] view."""
        kv = self.block[self.slot[layer_idx]]
        return kv[0], kv[1]

    def begin_step(self, positions):
        """Positions of the tokens about to run; every sequence's length becomes the last
        position + 1 (device ops only, so the step can be captured)."""
        self.positions = positions
        self.lengths.copy_((positions[-1:] + 1).to(torch.int32).expand(self.batch))

    def write(self, layer_idx, key, value):
        """Writes key/value [B, Hkv, S, D] of the current positions into the layer's pages."""
        k, v = self.pages(layer_idx)
        write_pages(key, value, k, v, self.tables, self.positions)

    def clear(self):
        self.lengths.zero_()


class HybridCache:
    """transformers cache protocol over the KV pool plus the linear-attention states."""

    def __init__(self, config, batch, capacity, device):
        kinds = list(config.layer_types)
        full = [i for i, kind in enumerate(kinds) if kind == "full_attention"]
        self.pool = PagedKVPool(full, batch, capacity, config.num_key_value_heads,
                                config.head_dim, device)
        # transformers reads per-layer linear-attention states as cache.layers[i]
        self.layers = [LinearAttentionLayer() if kind == "linear_attention" else None
                       for kind in kinds]
        self.linear = {i: layer for i, layer in enumerate(self.layers) if layer is not None}
        self.num_layers = len(kinds)
        self.phase = "prefill"

    def __len__(self):
        return self.num_layers

    # linear-attention layers
    def has_previous_state(self, layer_idx=None, state_idx=None):
        flags = self.linear[layer_idx].has_previous_state
        return all(flags.values()) if state_idx is None else flags[state_idx]

    def update_conv_state(self, conv_states, layer_idx, **kwargs):
        return self.linear[layer_idx].update_conv_state(conv_states, 0, **kwargs)

    def update_recurrent_state(self, recurrent_states, layer_idx, **kwargs):
        return self.linear[layer_idx].update_recurrent_state(recurrent_states, 0)

    def state_tensors(self):
        """Every linear-attention state tensor that exists (fixed addresses)."""
        found = []
        for layer in self.linear.values():
            for states in (layer.conv_states, layer.recurrent_states):
                found.extend(t for t in states.values() if t is not None)
        return found

    # full-attention layers
    def update(self, key, value, layer_idx, cache_kwargs=None):
        """Pages the chunk; prefill attends to the chunk itself, decode to the pages."""
        self.pool.write(layer_idx, key, value)
        return key, value

    def get_seq_length(self, layer_idx=0):
        return 0

    @torch.inference_mode()
    def reset(self):
        self.phase = "prefill"
        self.pool.clear()
        for layer in self.linear.values():
            layer.reset()


def _prefill_attention(query, key, value, scaling):
    """Causal GQA attention in float32 with contiguous operands; query [B, Hq, S, D] bf16,
    returns [B, S, Hq, D]."""
    s = query.shape[2]
    group = query.shape[1] // key.shape[1]
    q = query.float()
    k = key.float().repeat_interleave(group, dim=1).transpose(-1, -2).contiguous()
    v = value.float().repeat_interleave(group, dim=1).contiguous()
    scores = torch.matmul(q, k) * scaling
    future = torch.ones(s, s, dtype=torch.bool, device=query.device).triu(1)
    probs = scores.masked_fill(future, float("-inf")).softmax(-1)
    return torch.matmul(probs, v).transpose(1, 2).to(query.dtype)


def _dense_decode(q, k_pages, v_pages, tables, lengths, scaling):
    """float32 decode over the gathered pages (reads lengths on the host)."""
    out = torch.zeros_like(q)
    group = q.shape[1] // k_pages.shape[2]
    flat_k = k_pages.view(-1, *k_pages.shape[2:])
    flat_v = v_pages.view(-1, *v_pages.shape[2:])
    for b, length in enumerate(lengths.tolist()):
        if length == 0:
            continue
        pos = torch.arange(length, device=q.device)
        slots = tables[b, pos // PAGE].long() * PAGE + pos % PAGE
        k = flat_k[slots].float().repeat_interleave(group, dim=1).permute(1, 2, 0).contiguous()
        v = flat_v[slots].float().repeat_interleave(group, dim=1).permute(1, 0, 2).contiguous()
        scores = torch.matmul(q[b].float().unsqueeze(1), k) * scaling      # [Hq, 1, n]
        out[b] = torch.matmul(scores.softmax(-1), v).squeeze(1).to(q.dtype)
    return out


def _attention(module, query, key, value, attention_mask, scaling, dropout=0.0, **kwargs):
    if attention_mask is not None or dropout:
        raise ValueError("the hybrid runner supports unpadded inference batches only")
    runner = module.paged_decode_session
    cache = runner.cache
    if cache.phase == "prefill":
        return _prefill_attention(query, key, value, scaling), None
    q = query.squeeze(2)
    pool = cache.pool
    k, v = pool.pages(module.layer_idx)
    if runner.backend == "hip_matched":
        out = matched_decode(q, k, v, pool.tables, pool.lengths, resources=runner.resources,
                             scale=scaling)
    elif runner.backend == "torch":
        out = _dense_decode(q, k, v, pool.tables, pool.lengths, scaling)
    else:
        out = paged_decode(q, k, v, pool.tables, pool.lengths, resources=runner.resources,
                           backend=runner.backend, scale=scaling)
    if runner.attention_observer is not None:
        runner.attention_observer(module, q, k, v, out)
    return out.unsqueeze(1), None


AttentionInterface.register("paged_decode_lab_hip", _attention)


class DecodeStepGraph:
    """One decode step as a hipGraph; token and position come from static buffers."""

    def __init__(self, runner):
        self.runner = runner
        self.tokens = torch.zeros(runner.batch, 1, dtype=torch.long, device=runner.device)
        self.position = torch.zeros(1, dtype=torch.long, device=runner.device)
        self.graph = None
        self.logits = None

    def _load(self, token, position):
        self.tokens.copy_(token.view(-1, 1))
        self.position.fill_(position)

    @torch.inference_mode()
    def capture(self, token, position):
        """Captures the step at the current cache state and leaves that state as it was.
        The warm-up steps write the same KV rows the real step will write again."""
        runner, dev = self.runner, self.runner.device
        states = runner.cache.state_tensors()
        saved = [t.clone() for t in states]
        self._load(token, position)
        side = torch.cuda.Stream(device=dev)
        side.wait_stream(torch.cuda.current_stream(dev))
        with torch.cuda.stream(side):
            for _ in range(2):
                runner._forward(self.tokens, self.position)
            for t, s in zip(states, saved):
                t.copy_(s)
        torch.cuda.current_stream(dev).wait_stream(side)
        torch.cuda.synchronize(dev)
        del saved
        # Capture begins outside inference mode: torch registers its generators' graph
        # state when a capture begins, and tensors made in inference mode could not be
        # updated by later captures made outside it.
        with torch.inference_mode(False):
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph):
                self.logits = runner._forward(self.tokens, self.position)
        self.graph = graph

    def run(self, token, position):
        self._load(token, position)
        self.graph.replay()
        return self.logits


class HybridRunner:
    """Fixed-batch greedy generation over the paged decode path (the reference's
    HybridRunner, hybrid.py:104-228, for random-init weights)."""

    def __init__(self, config=None, *, model=None, backend="hip_matched", mode="eager", batch=1,
                 max_context=2048, device="cuda", seed=0):
        validate_hybrid_options(backend, mode, batch, max_context)
        self.backend, self.mode, self.batch = backend, mode, batch
        self.device = torch.device(device)
        if self.device.type != "cuda":
            raise ValueError("the hybrid runner requires a GPU device")
        self.max_context = max_context
        self.attention_observer = None
        self.model = model if model is not None else random_init_model(
            config if config is not None else decoder_config(), self.device, seed)
        self.text = self.model.model
        cfg = self.text.config
        self.spec = DecodeSpec(batch, cfg.num_attention_heads, cfg.num_key_value_heads,
                               cfg.head_dim, max_context)
        self.cache = HybridCache(cfg, batch, max_context, self.device)
        self.resources = allocate_hybrid_resources(self.spec, self.device, backend)
        self.attention_modules = [layer.self_attn for layer in self.text.layers
                                  if layer.block_type == "full_attention"]
        for module in self.attention_modules:
            module.config._attn_implementation = "paged_decode_lab_hip"
        self.step_graph = DecodeStepGraph(self) if mode == "graph" else None

    @torch.inference_mode()
    def _forward(self, tokens, positions):
        """Logits of the last token; tokens [B, S] at ``positions`` [S] (device tensors)."""
        # Several runners may share one model: the attention layers serve whichever
        # runner is running (a graph keeps the bindings it was captured with).
        for module in self.attention_modules:
            module.paged_decode_session = self
        with torch.device(self.device):
            self.cache.pool.begin_step(positions)
            hidden = self.text.embed_tokens(tokens)
            rope = self.text.rotary_emb(hidden, positions.view(1, 1, -1).expand(3, self.batch, -1))
            for layer in self.text.layers:
                hidden = layer(hidden, position_embeddings=rope, attention_mask=None,
                               past_key_values=self.cache, use_cache=True)
            return self.model.lm_head(self.text.norm(hidden)[:, -1])

    @torch.inference_mode()
    def prefill(self, token_rows):
        """Resets the cache, runs the prompt [B][S] in one forward and leaves the cache in
        its decode phase; returns the last position's logits."""
        self.cache.reset()
        tokens = torch.as_tensor(token_rows, dtype=torch.long, device=self.device)
        logits = self._forward(tokens, torch.arange(tokens.shape[1], device=self.device))
        self.cache.phase = "decode"
        return logits

    @torch.inference_mode()
    def decode_step(self, token, position):
        """Logits after feeding ``token`` [B] at ``position`` (eager or graph replay)."""
        if self.step_graph is None:
            return self._forward(token.view(-1, 1),
                                 torch.full((1,), position, dtype=torch.long, device=self.device))
        if self.step_graph.graph is None:
            self.step_graph.capture(token, position)
        return self.step_graph.run(token, position)

    @torch.inference_mode()
    def generate(self, prompts, output_tokens=32, *, forced=None, observe=False, timing=False):
        """Greedy decoding of ``output_tokens`` tokens after equally long prompts.

        The first token comes from the prefill logits, each later one from a decode step
        fed the previous token.  With ``forced`` (one batch vector per output token), step
        s feeds ``forced[s]`` instead of the prediction, so two backends can be compared
        logit by logit on one token sequence.  Returns the fed tokens (``token_ids``), the
        argmax predictions (``predicted_ids``), the per-step float32 logits on the host
        when ``observe`` and the decode steps' device times in ms when ``timing``."""
        if len(prompts) != self.batch or len({len(p) for p in prompts}) != 1:
            raise ValueError("fixed batch requires equally sized, unpadded token sequences")
        length = len(prompts[0])
        if length < 1 or output_tokens < 1 or length + output_tokens > self.max_context:
            raise ValueError("empty input/output or context capacity exceeded")
        fed = None
        if forced is not None:
            if len(forced) != output_tokens or any(len(row) != self.batch for row in forced):
                raise ValueError("forced tokens must provide one batch vector per step")
            fed = torch.as_tensor(forced, dtype=torch.long, device=self.device)
        logits = self.prefill(prompts)
        if self.step_graph is not None and self.step_graph.graph is None:
            # capture outside the timed steps, at the first decode position
            self.step_graph.capture(self._pick(logits, fed, 0)[1], length)
        tokens, predictions, saved, events = [], [], [], []
        for step in range(output_tokens):
            if step:
                if timing:
                    start, end = (torch.cuda.Event(enable_timing=True),
                                  torch.cuda.Event(enable_timing=True))
                    start.record()
                logits = self.decode_step(tokens[-1], length + step - 1)
                if timing:
                    end.record()
                    events.append((start, end))
            if observe:
                host = logits.float().cpu()
                if not torch.isfinite(host).all():
                    raise FloatingPointError(f"non-finite logits at decode step {step}")
                saved.append(host)
            predicted, token = self._pick(logits, fed, step)
            predictions.append(predicted)
            tokens.append(token)
        torch.cuda.synchronize(self.device)
        return {"token_ids": torch.stack(tokens, 1).cpu().tolist(),
                "predicted_ids": torch.stack(predictions, 1).cpu().tolist(),
                "logits": saved, "decode_ms": [a.elapsed_time(b) for a, b in events]}

    @staticmethod
    def _pick(logits, fed, step):
        predicted = logits.argmax(-1)
        return predicted, (predicted if fed is None else fed[step])

    def describe(self):
        """Geometry, plan and workspace of this runner (a host-side record)."""
        matched = self.backend == "hip_matched"
        if matched:
            workspace = (self.resources.partials.numel() + self.resources.lse.numel()) * 4
        elif self.backend == "hip_splitk":
            workspace = self.spec.split_workspace_bytes
        else:
            workspace = 0
        pool = self.cache.pool
        return {"backend": self.backend, "mode": self.mode, "batch": self.batch,
                "max_context": self.max_context,
                "splitkv_plan": dataclasses.asdict(self.resources.plan) if matched else None,
                "workspace_bytes": workspace,
                "full_attention_layers": len(pool.slot),
                "linear_attention_layers": len(self.cache.linear),
                "heads": self.spec.num_heads, "kv_heads": self.spec.num_kv_heads,
                "head_dim": self.spec.head_dim, "pages_per_full_layer": self.batch * pool.width,
                "graph_scope": "decode step: every layer (KV write, attention, linear-attention "
                               "state updates) and the lm_head; not the prefill or token choice"}
