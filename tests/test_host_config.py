"""Host-side model configuration: the transformers configs the forward
accepts, and the ones it refuses rather than run with math it does not
carry (projection biases, scaled RoPE).  No GPU needed."""
import pytest
from transformers import LlamaConfig

from lm.model import SMOLLM2_1_7B, shape_from_hf_config


def small(**kw):
    return LlamaConfig(vocab_size=256, hidden_size=64, num_hidden_layers=2, num_attention_heads=4,
                       num_key_value_heads=2, intermediate_size=128, **kw)


def test_plain_llama_config_converts():
    shape = shape_from_hf_config(small(rope_theta=130000.0, rms_norm_eps=1e-5))
    assert (shape.hidden_size, shape.num_attention_heads, shape.num_key_value_heads, shape.head_dim) == (64, 4, 2, 16)
    assert shape.rope_theta == 130000.0 and shape.rms_norm_eps == 1e-5


def test_smollm2_shape_round_trips_through_a_config():
    s = SMOLLM2_1_7B
    cfg = LlamaConfig(vocab_size=s.vocab_size, hidden_size=s.hidden_size, num_hidden_layers=s.num_hidden_layers,
                      num_attention_heads=s.num_attention_heads, num_key_value_heads=s.num_key_value_heads,
                      intermediate_size=s.intermediate_size, rope_theta=s.rope_theta, rms_norm_eps=s.rms_norm_eps,
                      tie_word_embeddings=True, max_position_embeddings=s.max_position_embeddings)
    assert shape_from_hf_config(cfg) == s


@pytest.mark.parametrize("kw", [{"attention_bias": True}, {"mlp_bias": True}])
def test_projection_biases_are_refused(kw):
    with pytest.raises(NotImplementedError, match="bias"):
        shape_from_hf_config(small(**kw))


def test_scaled_rope_is_refused():
    cfg = small(max_position_embeddings=16384, rope_scaling={
        "rope_type": "llama3", "factor": 8.0, "low_freq_factor": 1.0, "high_freq_factor": 4.0,
        "original_max_position_embeddings": 8192})
    with pytest.raises(NotImplementedError, match="llama3"):
        shape_from_hf_config(cfg)


def test_qwen2_is_refused():
    from transformers import Qwen2Config

    cfg = Qwen2Config(vocab_size=256, hidden_size=64, num_hidden_layers=2, num_attention_heads=4,
                      num_key_value_heads=2, intermediate_size=128)
    with pytest.raises(NotImplementedError, match="qwen2"):
        shape_from_hf_config(cfg)
