"""Oracle of lm/forward.py: the cached Llama forward with the gather copy and
SDPA, written over a Hugging Face-named state dict so it runs on any weights
(test infrastructure, see oracle/__init__.py).  The layer math follows
transformers' Llama modules as lm/forward.py:51-65 calls them."""
from dataclasses import dataclass

import torch
import torch.nn.functional as F


@dataclass(frozen=True)
class Config:
    vocab_size: int
    hidden_size: int
    num_hidden_layers: int
    num_attention_heads: int
    num_key_value_heads: int
    intermediate_size: int
    head_dim: int
    rms_norm_eps: float
    rope_theta: float
    tie_word_embeddings: bool = True


class Model:
    """Weights (HF names) on the CPU plus the fp32 head copy (lm/forward.py:71-84)."""

    def __init__(self, config: Config, state: dict[str, torch.Tensor]) -> None:
        self.config = config
        self.w = state
        head = state["model.embed_tokens.weight"] if config.tie_word_embeddings else state["lm_head.weight"]
        self.head_wide = head.to(torch.promote_types(head.dtype, torch.float32))
        d = config.head_dim
        self.inv_freq = 1.0 / (config.rope_theta ** (torch.arange(0, d, 2, dtype=torch.int64).float() / d))
        self.scaling = d ** -0.5

    @property
    def dtype(self):
        return self.w["model.embed_tokens.weight"].dtype


def rms_norm(x, weight, eps):
    """transformers LlamaRMSNorm.forward"""
    h = x.to(torch.float32)
    h = h * torch.rsqrt(h.pow(2).mean(-1, keepdim=True) + eps)
    return weight * h.to(x.dtype)


def rotary(model: Model, hidden, positions):
    """transformers LlamaRotaryEmbedding.forward: fp32 angles, cast to the input dtype"""
    freqs = positions.float()[..., None] * model.inv_freq[None, None, :]
    emb = torch.cat((freqs, freqs), dim=-1)
    return emb.cos().to(hidden.dtype), emb.sin().to(hidden.dtype)


def rotate_half(x):
    x1, x2 = x[..., : x.shape[-1] // 2], x[..., x.shape[-1] // 2:]
    return torch.cat((-x2, x1), dim=-1)


def apply_rotary(q, k, cos, sin):
    """transformers apply_rotary_pos_emb with unsqueeze_dim=1"""
    cos, sin = cos.unsqueeze(1), sin.unsqueeze(1)
    return q * cos + rotate_half(q) * sin, k * cos + rotate_half(k) * sin


@torch.no_grad()
def forward(model: Model, cache, seq_ids, input_ids, n_new, last_only=False):
    """lm/forward.py:21-68"""
    cfg, w = model.config, model.w
    slots = cache.append(seq_ids, n_new)
    b, t = input_ids.shape
    positions = slots.past[:, None] + torch.arange(t)
    keys = torch.arange(slots.read.shape[1])
    allowed = (keys[None, None, :] <= positions[:, :, None]) & (keys[None, None, :] < slots.total[:, None, None])
    mask = allowed[:, None, :, :]
    hidden = F.embedding(input_ids, w["model.embed_tokens.weight"])
    cos, sin = rotary(model, hidden, positions)
    d = cfg.head_dim
    for i in range(cfg.num_hidden_layers):
        p = f"model.layers.{i}."
        x = rms_norm(hidden, w[p + "input_layernorm.weight"], cfg.rms_norm_eps)
        q = F.linear(x, w[p + "self_attn.q_proj.weight"]).view(b, t, -1, d).transpose(1, 2)
        k = F.linear(x, w[p + "self_attn.k_proj.weight"]).view(b, t, -1, d).transpose(1, 2)
        v = F.linear(x, w[p + "self_attn.v_proj.weight"]).view(b, t, -1, d).transpose(1, 2)
        q, k = apply_rotary(q, k, cos, sin)
        cache.write(i, slots, k, v)
        k_all, v_all = cache.gather(i, slots)
        out = F.scaled_dot_product_attention(q, k_all, v_all, attn_mask=mask, scale=model.scaling, enable_gqa=True)
        hidden = hidden + F.linear(out.transpose(1, 2).reshape(b, t, -1), w[p + "self_attn.o_proj.weight"])
        x = rms_norm(hidden, w[p + "post_attention_layernorm.weight"], cfg.rms_norm_eps)
        mlp = F.linear(F.silu(F.linear(x, w[p + "mlp.gate_proj.weight"])) * F.linear(x, w[p + "mlp.up_proj.weight"]),
                       w[p + "mlp.down_proj.weight"])
        hidden = hidden + mlp
    if last_only:
        hidden = hidden[torch.arange(b), slots.total - slots.past - 1]
    return logits(model, rms_norm(hidden, w["model.norm.weight"], cfg.rms_norm_eps))


def logits(model: Model, hidden):
    """lm/forward.py:71-84"""
    return F.linear(hidden.to(model.head_wide.dtype), model.head_wide)


def attention(q, k_all, v_all, past, total, scaling):
    """The attention step of lm/forward.py:44-49,63 on gathered K/V:
    q [B, H, T, d], k_all/v_all [B, Hkv, S, d], past/total [B]."""
    b, _, t, _ = q.shape
    positions = past[:, None] + torch.arange(t)
    keys = torch.arange(k_all.shape[2])
    allowed = (keys[None, None, :] <= positions[:, :, None]) & (keys[None, None, :] < total[:, None, None])
    return F.scaled_dot_product_attention(q, k_all, v_all, attn_mask=allowed[:, None], scale=scaling,
                                          enable_gqa=True)
