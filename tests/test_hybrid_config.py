"""Host-side checks of the end-to-end decoder runner (CPU only)."""
import pytest

from paged_decode import hybrid as H


def test_decoder_geometry():
    cfg = H.decoder_config()
    assert (cfg.num_hidden_layers, cfg.hidden_size, cfg.vocab_size) == (24, 2048, 151936)
    assert (cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim) == (8, 2, 256)
    assert cfg.layer_types.count("full_attention") == 6
    assert cfg.layer_types[3] == "full_attention" and cfg.layer_types[0] == "linear_attention"


@pytest.mark.parametrize("args,match", [
    (("flash_attn", "eager", 1, 100), "backend"), (("hip_matched", "compiled", 1, 100), "mode"),
    (("torch", "graph", 1, 100), "eager"), (("hip_matched", "eager", 0, 100), "batch"),
    (("hip_base", "graph", 1, 2), "max_context")])
def test_options_are_rejected(args, match):
    with pytest.raises(ValueError, match=match):
        H.validate_hybrid_options(*args)
