"""The end-to-end decoder at its full size: 24 layers (6 of them full attention with
Hq 8 / Hkv 2 / D 256), hidden 2048, vocab 151936, random-init bf16 weights with
std 0.02, batch 1, prompts of 512 and 2048 random token ids, 64 output tokens.

Checks, for each prompt length:
* graph replay produces the same 64 greedy tokens as eager execution, with the
  same logits;
* inside the model, every decode call of the matched HIP operator (6 layers x 63
  steps, real activations) is within 2e-2 of float32 dense attention on the same
  query, pages and length, and sampled calls pass the oracle's one-ulp gate;
* teacher-forced on the float32 backend's greedy tokens, the matched HIP decode's
  logits stay within the network's one-ulp noise floor of the float32 backend's;
* the last decode step's logits match one prefill over the prompt and the
  generated tokens as closely as the float32 backend's do.

The noise floor.  A bf16 network 24 layers deep amplifies a one-ulp change of an
attention output into logit changes of about 0.1 (logits here span about +-5).
The floor is measured, not assumed: the float32 backend is run a second time with
its attention outputs stochastically rounded to bf16 (one bf16 ulp of unbiased
noise on every output), on the same forced tokens.  Any decode attention that is
not bit-identical to the float32 backend's lands at that level, so the HIP logits
must stay within 1.5x of it (max and median over the 64 steps); a protocol
mistake of more than an ulp lands far above it.  Per-step maxima are recorded
for the parity summary at the end of the run.
"""
import numpy as np
import pytest
import torch

if not torch.cuda.is_available():
    pytest.skip("needs an MI355X GPU", allow_module_level=True)

from gpu_cases import assert_within_one_ulp, to_np
from oracle import matched as OM
from paged_decode import hybrid as H
from parity import record

pytestmark = pytest.mark.gpu
OUTPUT_TOKENS = 64
VOCAB = 151936
CAPACITY = 2048 + OUTPUT_TOKENS
FLOOR_MARGIN = 1.5


@pytest.fixture(scope="module")
def model():
    cfg = H.decoder_config()
    assert (cfg.num_hidden_layers, cfg.hidden_size, cfg.vocab_size) == (24, 2048, VOCAB)
    return H.random_init_model(cfg, "cuda", seed=0)


@pytest.fixture(scope="module")
def runners(model):
    return {mode: H.HybridRunner(model=model, backend="hip_matched", mode=mode,
                                 max_context=CAPACITY)
            for mode in ("eager", "graph")}


@pytest.fixture(scope="module")
def eager_runs():
    return {}


def prompt(length):
    gen = torch.Generator().manual_seed(length)
    return [torch.randint(0, VOCAB, (length,), generator=gen).tolist()]


def eager_run(runners, eager_runs, plen):
    if plen not in eager_runs:
        eager_runs[plen] = runners["eager"].generate(prompt(plen), OUTPUT_TOKENS, observe=True)
    return eager_runs[plen]


def step_diffs(a, b):
    return [float((x - y).abs().max()) for x, y in zip(a["logits"], b["logits"])]


def dense_decode_one_ulp_noise(q, k_pages, v_pages, tables, lengths, scaling):
    """float32 decode whose outputs are stochastically rounded to bf16: unbiased noise of
    one bf16 ulp on every output (seeded by the length, so runs repeat)."""
    out = torch.zeros_like(q)
    group = q.shape[1] // k_pages.shape[2]
    flat_k = k_pages.view(-1, *k_pages.shape[2:])
    flat_v = v_pages.view(-1, *v_pages.shape[2:])
    for b, length in enumerate(lengths.tolist()):
        if length == 0:
            continue
        gen = torch.Generator(device=q.device).manual_seed(length)
        pos = torch.arange(length, device=q.device)
        slots = tables[b, pos // 256].long() * 256 + pos % 256
        k = flat_k[slots].float().repeat_interleave(group, dim=1).permute(1, 2, 0).contiguous()
        v = flat_v[slots].float().repeat_interleave(group, dim=1).permute(1, 0, 2).contiguous()
        probs = (torch.matmul(q[b].float().unsqueeze(1), k) * scaling).softmax(-1)
        exact = torch.matmul(probs, v).squeeze(1).contiguous()
        noise = torch.randint(0, 1 << 16, exact.shape, device=q.device, generator=gen,
                              dtype=torch.int32)
        out[b] = ((exact.view(torch.int32) + noise) & ~0xFFFF).view(torch.float32).to(q.dtype)
    return out


@pytest.mark.parametrize("plen", [512, 2048])
def test_graph_tokens_equal_eager(runners, eager_runs, plen):
    eager = eager_run(runners, eager_runs, plen)
    graph = runners["graph"].generate(prompt(plen), OUTPUT_TOKENS, observe=True)
    assert len(graph["token_ids"][0]) == OUTPUT_TOKENS
    assert graph["token_ids"] == eager["token_ids"]
    diff = max(step_diffs(graph, eager))
    record(f"decoder 24L prompt {plen}: graph vs eager logits", max_abs=diff)
    assert diff < 1e-3


@pytest.mark.parametrize("plen", [512, 2048])
def test_operator_parity_inside_the_model(runners, plen):
    runner = runners["eager"]
    dense_max, sampled = [0.0], []

    def observe(module, q, k, v, out):
        pool = runner.cache.pool
        dense = H._dense_decode(q, k, v, pool.tables, pool.lengths, module.scaling)
        dense_max[0] = max(dense_max[0], float((out.float() - dense.float()).abs().max()))
        length = int(pool.lengths[0])
        if length in (plen + 1, plen + OUTPUT_TOKENS - 1):
            sampled.append((to_np(q), to_np(k), to_np(v), pool.tables.cpu().numpy(),
                            pool.lengths.cpu().numpy(), to_np(out), module.scaling))

    runner.attention_observer = observe
    try:
        runner.generate(prompt(plen), OUTPUT_TOKENS)
    finally:
        runner.attention_observer = None
    assert len(sampled) == 2 * 6
    record(f"decoder 24L prompt {plen}: matched decode vs float32 dense in the model",
           max_abs_vs_dense=dense_max[0])
    assert dense_max[0] < 2e-2
    plan = runner.resources.plan
    for q, k, v, table, lengths, out, scale in sampled:
        expected, _, _, bound, _ = OM.matched_decode_with_bounds(
            q, k, v, table, lengths, plan.splits, plan.tokens_per_split, plan.tile_tokens,
            plan.lse_lanes, scale)
        assert_within_one_ulp(out, expected, f"decoder layer call at length {lengths[0]}", bound)


@pytest.mark.parametrize("plen", [512, 2048])
def test_logits_within_the_one_ulp_noise_floor(model, runners, monkeypatch, plen):
    ref_runner = H.HybridRunner(model=model, backend="torch", max_context=CAPACITY)
    ref = ref_runner.generate(prompt(plen), OUTPUT_TOKENS, observe=True)
    forced = [[t] for t in ref["token_ids"][0]]
    hip = runners["eager"].generate(prompt(plen), OUTPUT_TOKENS, observe=True, forced=forced)
    with monkeypatch.context() as patch:
        patch.setattr(H, "_dense_decode", dense_decode_one_ulp_noise)
        noisy = ref_runner.generate(prompt(plen), OUTPUT_TOKENS, observe=True, forced=forced)
    d_hip, d_floor = step_diffs(hip, ref), step_diffs(noisy, ref)
    assert d_hip[0] == 0.0 and d_floor[0] == 0.0     # step 0 comes from the same prefill
    agree = sum(p == r for p, r in zip(hip["predicted_ids"][0], ref["predicted_ids"][0]))
    record(f"decoder 24L prompt {plen}: matched vs float32 attention logits",
           max_abs=max(d_hip), noise_floor_max_abs=max(d_floor),
           argmax_agreement=agree / OUTPUT_TOKENS)
    print(f"prompt {plen}: |logit diff| max {max(d_hip):.4f} median {np.median(d_hip):.4f}; "
          f"one-ulp floor max {max(d_floor):.4f} median {np.median(d_floor):.4f}; "
          f"argmax agreement {agree}/{OUTPUT_TOKENS}")
    assert max(d_hip) <= FLOOR_MARGIN * max(d_floor)
    assert np.median(d_hip) <= FLOOR_MARGIN * np.median(d_floor)


@pytest.mark.parametrize("plen", [512, 2048])
def test_last_step_matches_a_full_prefill(model, runners, eager_runs, plen):
    eager = eager_run(runners, eager_runs, plen)
    tokens = prompt(plen)[0] + eager["token_ids"][0][:-1]
    diff = float((runners["eager"].prefill([tokens]).float().cpu() - eager["logits"][-1])
                 .abs().max())
    # the same comparison with float32 decode attention on the same tokens
    ref_runner = H.HybridRunner(model=model, backend="torch", max_context=CAPACITY)
    ref = ref_runner.generate(prompt(plen), OUTPUT_TOKENS, observe=True,
                              forced=[[t] for t in eager["token_ids"][0]])
    ref_diff = float((ref_runner.prefill([tokens]).float().cpu() - ref["logits"][-1])
                     .abs().max())
    record(f"decoder 24L prompt {plen}: last step vs re-prefill logits", max_abs=diff,
           float32_backend_max_abs=ref_diff)
    print(f"prompt {plen}: last step vs re-prefill {diff:.4f} (float32 attention {ref_diff:.4f})")
    assert diff <= FLOOR_MARGIN * ref_diff
