"""End-to-end decoding through the paged path (random-init Qwen3.5 geometry).

A small config (4 layers, one full-attention layer with Hq 8 / Hkv 2 / D 256)
keeps the test fast; the decode logits of the HIP backends are compared with
the float32 PyTorch reference backend and with a full re-prefill, and graph
replay with eager execution.
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


def run(model, backend, mode="eager", steps=6):
    runner = H.HybridRunner(model=model, backend=backend, mode=mode, max_context=600)
    return runner, runner.generate(PROMPT, output_tokens=steps, observe=True)


def test_hip_backends_match_the_torch_reference(model):
    _, ref = run(model, "torch")
    for backend in ("hip_matched", "hip_base", "hip_splitk"):
        _, out = run(model, backend)
        for step, (a, b) in enumerate(zip(out["logits"], ref["logits"])):
            assert (a - b).abs().max() < 2e-2, (backend, step, float((a - b).abs().max()))


def test_graph_replay_matches_eager(model):
    _, eager = run(model, "hip_matched", "eager")
    _, graph = run(model, "hip_matched", "graph")
    assert graph["token_ids"] == eager["token_ids"]
    for a, b in zip(graph["logits"], eager["logits"]):
        assert (a - b).abs().max() < 1e-3


def test_decode_matches_a_full_prefill(model):
    runner, out = run(model, "hip_matched", steps=4)
    tokens = PROMPT[0] + out["token_ids"][0][:-1]
    runner.cache.reset()
    with torch.inference_mode():
        logits = runner._forward(torch.tensor([tokens], device="cuda"),
                                 torch.arange(len(tokens), device="cuda"))
    assert (logits.float().cpu() - out["logits"][-1]).abs().max() < 2e-2


def test_options_are_validated():
    with pytest.raises(ValueError, match="backend"):
        H.validate_hybrid_options("flash_attn", "eager", 1, 100)
    with pytest.raises(ValueError, match="eager"):
        H.validate_hybrid_options("torch", "graph", 1, 100)
