"""Tiny Llama models shared by the tests (CPU construction, seeded)."""
import hashlib

import torch


def reference_tiny(seed: int = 0, dtype=torch.float64):
    """The reference's tiny model recipe (lm/load.py:124-141): 2 layers,
    hidden 64, 4 query / 2 KV heads, vocab 256, transformers' default init
    after torch.manual_seed(seed)."""
    from transformers import LlamaConfig, LlamaForCausalLM

    config = LlamaConfig(vocab_size=256, hidden_size=64, intermediate_size=128, num_hidden_layers=2,
                         num_attention_heads=4, num_key_value_heads=2, max_position_embeddings=1024,
                         attn_implementation="sdpa")
    torch.manual_seed(seed)
    return LlamaForCausalLM(config).to(dtype).eval()


def tiny64(seed: int = 0, dtype=torch.float32, layers: int = 2):
    """A tiny Llama with head_dim 64 (what the attention kernel implements):
    hidden 256, 4 query / 2 KV heads, MLP 512, vocab 256."""
    from transformers import LlamaConfig, LlamaForCausalLM

    config = LlamaConfig(vocab_size=256, hidden_size=256, intermediate_size=512, num_hidden_layers=layers,
                         num_attention_heads=4, num_key_value_heads=2, head_dim=64, max_position_embeddings=2048,
                         attn_implementation="sdpa", rope_theta=10000.0)
    torch.manual_seed(seed)
    model = LlamaForCausalLM(config).to(dtype).eval()
    # transformers initialises with std 0.02; widen the embeddings and the
    # first layer (x3) so greedy choices are well separated, and the later
    # layers less (x1.5) so a first-layer early exit agrees with the target
    # about half the time (acceptance ~0.5 in the loop)
    with torch.no_grad():
        for name, p in model.named_parameters():
            if p.dim() == 2:
                late = name.startswith("model.layers.") and not name.startswith("model.layers.0.")
                p.mul_(1.5 if late else 3.0)
    return model


def early_exit(model, n_layers: int = 1):
    import copy

    draft = copy.deepcopy(model)
    draft.__dict__.pop("_specdec_llama", None)  # a conversion cached on the target is not the draft's
    draft.model.layers = draft.model.layers[:n_layers]
    draft.config.num_hidden_layers = n_layers
    return draft


def weights_sha(model) -> str:
    h = hashlib.sha256()
    for name, t in sorted(model.state_dict().items()):
        h.update(name.encode())
        h.update(t.detach().double().numpy().tobytes())
    return h.hexdigest()


def random_prompts(n: int, vocab: int, seed: int, low: int = 3, high: int = 20):
    gen = torch.Generator().manual_seed(seed)
    lengths = torch.randint(low, high, (n,), generator=gen).tolist()
    return [torch.randint(0, vocab, (m,), generator=gen).tolist() for m in lengths]


def oracle_model(hf_model):
    """oracle.forward.Model over an HF model's weights (CPU)."""
    import oracle.forward as of

    c = hf_model.config
    head_dim = getattr(c, "head_dim", None) or c.hidden_size // c.num_attention_heads
    theta = getattr(c, "rope_theta", None) or c.rope_parameters["rope_theta"]
    cfg = of.Config(c.vocab_size, c.hidden_size, c.num_hidden_layers, c.num_attention_heads, c.num_key_value_heads,
                    c.intermediate_size, head_dim, c.rms_norm_eps, float(theta), bool(c.tie_word_embeddings))
    return of.Model(cfg, {k: v.detach() for k, v in hf_model.state_dict().items()})
