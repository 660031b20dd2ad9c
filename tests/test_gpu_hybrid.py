"""End-to-end decoding through the paged path (random-init Qwen3.5 geometry, small).

A small config (4 layers, one full-attention layer with Hq 8 / Hkv 2 / D 256)
keeps these tests fast; tests/test_gpu_decoder_full.py runs the full 24-layer
geometry.  The decode logits of the HIP backends are compared with the float32
PyTorch backend on one teacher-forced token sequence, graph replay with eager
execution, and the last decode step with a full re-prefill.
"""
import pytest
import torch

if not torch.cuda.is_available():
    pytest.skip("needs an MI355X GPU", allow_module_level=True)

from paged_decode import hybrid as H

pytestmark = pytest.mark.gpu
PROMPT = [list(range(3, 300))]


@pytest.fixture(scope="module")
def model():
    cfg = H.decoder_config(num_hidden_layers=4, hidden_size=256, intermediate_size=512,
                           vocab_size=512, linear_num_key_heads=4, linear_key_head_dim=64,
                           linear_num_value_heads=4, linear_value_head_dim=64)
    return H.random_init_model(cfg, "cuda", seed=1)


def run(model, backend, mode="eager", steps=6, forced=None):
    runner = H.HybridRunner(model=model, backend=backend, mode=mode, max_context=600)
    return runner, runner.generate(PROMPT, output_tokens=steps, observe=True, forced=forced)


def test_hip_backends_match_the_torch_reference(model):
    _, ref = run(model, "torch")
    for backend in ("hip_matched", "hip_base", "hip_splitk"):
        _, out = run(model, backend, forced=[[t] for t in ref["token_ids"][0]])
        assert out["token_ids"] == ref["token_ids"]
        for step, (a, b) in enumerate(zip(out["logits"], ref["logits"])):
            assert (a - b).abs().max() < 2e-2, (backend, step, float((a - b).abs().max()))


def test_graph_replay_matches_eager(model):
    _, eager = run(model, "hip_matched", "eager")
    runner, graph = run(model, "hip_matched", "graph")
    assert graph["token_ids"] == eager["token_ids"]
    for a, b in zip(graph["logits"], eager["logits"]):
        assert (a - b).abs().max() < 1e-3
    # the graph captured by the first generation serves the next one
    captured = runner.step_graph.graph
    again = runner.generate(PROMPT, output_tokens=6, observe=True)
    assert runner.step_graph.graph is captured
    assert again["token_ids"] == eager["token_ids"]
    for a, b in zip(again["logits"], graph["logits"]):
        assert torch.equal(a, b)


def test_decode_matches_a_full_prefill(model):
    runner, out = run(model, "hip_matched", steps=4)
    tokens = PROMPT[0] + out["token_ids"][0][:-1]
    logits = runner.prefill([tokens])
    assert (logits.float().cpu() - out["logits"][-1]).abs().max() < 2e-2


def test_teacher_forcing_feeds_the_given_tokens(model):
    _, free = run(model, "hip_matched", steps=5)
    forced = [[(t + 7) % 512] for t in free["token_ids"][0]]
    _, out = run(model, "hip_matched", steps=5, forced=forced)
    assert out["token_ids"][0] == [row[0] for row in forced]
    # step 0 comes from the prefill, so its prediction is the free run's first token
    assert out["predicted_ids"][0][0] == free["token_ids"][0][0]
    with pytest.raises(ValueError, match="forced"):
        run(model, "hip_matched", steps=5, forced=forced[:4])


def test_attention_observer_sees_every_decode_call(model):
    runner = H.HybridRunner(model=model, backend="hip_matched", max_context=600)
    seen = []
    runner.attention_observer = lambda module, q, k, v, out: seen.append(
        (module.layer_idx, tuple(q.shape), bool(torch.isfinite(out).all())))
    runner.generate(PROMPT, output_tokens=3)
    full = [i for i, kind in enumerate(model.config.layer_types) if kind == "full_attention"]
    assert seen == [(i, (1, 8, 256), True) for _ in range(2) for i in full]


def test_options_are_validated():
    with pytest.raises(ValueError, match="backend"):
        H.validate_hybrid_options("flash_attn", "eager", 1, 100)
    with pytest.raises(ValueError, match="eager"):
        H.validate_hybrid_options("torch", "graph", 1, 100)
