"""Llama-architecture weights held as plain device tensors.

lm/forward.py runs on this container of weights: the q/k/v projections
are fused into one [(H + 2*Hkv)*d, hidden] weight and gate/up into one
[2*I, hidden] weight, so each layer is four GEMMs.  Weights use the
Hugging Face state-dict names on the way in (`from_state_dict`, `from_hf`),
so a transformers LlamaForCausalLM converts directly and a random-init model
can be compared against one.

RoPE tables are built the way transformers' LlamaRotaryEmbedding builds them
(inv_freq = 1 / theta^(arange(0, d, 2) / d) in fp32, angle = position *
inv_freq in fp32, then cos and sin), and kept in fp32 on the device.
"""
from __future__ import annotations

from dataclasses import dataclass, field

import torch

from specdec import ops


@dataclass(frozen=True)
class LlamaShape:
    vocab_size: int
    hidden_size: int
    num_hidden_layers: int
    num_attention_heads: int
    num_key_value_heads: int
    intermediate_size: int
    head_dim: int = 64
    rms_norm_eps: float = 1e-5
    rope_theta: float = 10000.0
    tie_word_embeddings: bool = True
    max_position_embeddings: int = 8192
    model_type: str = "llama"

    def replace(self, **kw) -> "LlamaShape":
        from dataclasses import replace

        return replace(self, **kw)


# SmolLM2 shapes (the target and draft of the benchmark)
SMOLLM2_1_7B = LlamaShape(vocab_size=49152, hidden_size=2048, num_hidden_layers=24, num_attention_heads=32,
                          num_key_value_heads=32, intermediate_size=8192, rope_theta=130000.0)
SMOLLM2_135M = LlamaShape(vocab_size=49152, hidden_size=576, num_hidden_layers=30, num_attention_heads=9,
                          num_key_value_heads=3, intermediate_size=1536, rope_theta=100000.0)


def hf_names(shape: LlamaShape) -> list[tuple[str, tuple[int, ...]]]:
    """(name, shape) of every weight, in a fixed order."""
    h, d, i = shape.hidden_size, shape.head_dim, shape.intermediate_size
    hq, hk = shape.num_attention_heads * d, shape.num_key_value_heads * d
    out = [("model.embed_tokens.weight", (shape.vocab_size, h))]
    for n in range(shape.num_hidden_layers):
        p = f"model.layers.{n}."
        out += [
            (p + "input_layernorm.weight", (h,)),
            (p + "self_attn.q_proj.weight", (hq, h)),
            (p + "self_attn.k_proj.weight", (hk, h)),
            (p + "self_attn.v_proj.weight", (hk, h)),
            (p + "self_attn.o_proj.weight", (h, hq)),
            (p + "post_attention_layernorm.weight", (h,)),
            (p + "mlp.gate_proj.weight", (i, h)),
            (p + "mlp.up_proj.weight", (i, h)),
            (p + "mlp.down_proj.weight", (h, i)),
        ]
    out.append(("model.norm.weight", (h,)))
    if not shape.tie_word_embeddings:
        out.append(("lm_head.weight", (shape.vocab_size, h)))
    return out


def random_state_dict(shape: LlamaShape, seed: int, device, dtype: torch.dtype = torch.bfloat16,
                      std: float = 0.02) -> dict[str, torch.Tensor]:
    """Seeded random init: matrices ~ N(0, std^2) (drawn in fp32, then cast),
    norm weights = 1 (as transformers initialises RMSNorm).  Tensor n uses a
    generator seeded with seed * 1000003 + n on `device`."""
    device = torch.device(device)
    out = {}
    for n, (name, shp) in enumerate(hf_names(shape)):
        if len(shp) == 1:
            out[name] = torch.ones(shp, dtype=dtype, device=device)
            continue
        gen = torch.Generator(device=device).manual_seed(seed * 1000003 + n)
        w = torch.empty(shp, dtype=torch.float32, device=device)
        w.normal_(0.0, std, generator=gen)
        out[name] = w.to(dtype)
    return out


def perturbed_truncation(state: dict[str, torch.Tensor], shape: LlamaShape, n_layers: int, noise: float,
                         seed: int) -> tuple[dict[str, torch.Tensor], LlamaShape]:
    """A draft made of the target's first `n_layers` layers (embeddings, final
    norm and head shared) plus N(0, noise^2) on every matrix of those layers."""
    small = shape.replace(num_hidden_layers=n_layers)
    out = {}
    for n, (name, shp) in enumerate(hf_names(small)):
        w = state[name]
        if len(shp) == 2 and name.startswith("model.layers.") and noise > 0:
            gen = torch.Generator(device=w.device).manual_seed(seed * 1000003 + n)
            z = torch.empty(shp, dtype=torch.float32, device=w.device).normal_(0.0, noise, generator=gen)
            w = (w.float() + z).to(w.dtype)
        out[name] = w
    return out, small


@dataclass
class Layer:
    """One decoder layer.  The two RMSNorm weights are folded into the
    columns of the projections that read the norms' outputs (W diag(ln), one
    rounding to the weight dtype; exact for the unit weights of a fresh
    model), because the forward projects the unnormalised residual stream
    and finishes each norm after the projection: RMSNorm(x) @ W^T =
    rsqrt(mean(x^2) + eps) * (x @ (W diag(ln))^T)."""
    ln1: torch.Tensor
    wqkv: torch.Tensor  # q/k/v [(H + 2 Hkv) d, hidden], ln1 folded in
    wo: torch.Tensor
    ln2: torch.Tensor
    wgu: torch.Tensor  # gate/up [2 * intermediate, hidden], ln2 folded in
    wd: torch.Tensor
    # the same four in the decode-sized projections' tiled layout
    # (ops.tile_weight: the same bits, contiguous loads), made for bf16
    # weights on the GPU; None otherwise (prompt-sized GEMMs read the above)
    wqkv_t: torch.Tensor | None = field(default=None, repr=False)
    wo_t: torch.Tensor | None = field(default=None, repr=False)
    wgu_t: torch.Tensor | None = field(default=None, repr=False)
    wd_t: torch.Tensor | None = field(default=None, repr=False)

    def __post_init__(self):
        def tiled(w: torch.Tensor) -> torch.Tensor | None:
            if not (w.is_cuda and w.dtype == torch.bfloat16 and w.dim() == 2 and w.shape[0] % 16 == 0
                    and w.shape[1] % 32 == 0):
                return None
            return ops.tile_weight(w)
        if self.wqkv_t is None:
            self.wqkv_t, self.wo_t, self.wgu_t, self.wd_t = (tiled(w) for w in (self.wqkv, self.wo, self.wgu, self.wd))


def fold_norm(w: torch.Tensor, ln: torch.Tensor) -> torch.Tensor:
    """W diag(ln): the norm weight multiplied into W's columns, in fp32 or
    wider, then rounded once to W's dtype."""
    wide = torch.promote_types(w.dtype, torch.float32)
    return (w.to(wide) * ln.to(wide)).to(w.dtype).contiguous()


@dataclass
class Llama:
    config: LlamaShape
    embed: torch.Tensor
    layers: list[Layer]
    norm: torch.Tensor
    lm_head: torch.Tensor
    # lm_head as the output projection reads it: bf16/fp16 weights on the GPU
    # as stored (the GEMM accumulates in and writes fp32), else an fp32 (or
    # wider) copy made once
    head_wide: torch.Tensor
    rope_cos: torch.Tensor = field(repr=False)
    rope_sin: torch.Tensor = field(repr=False)
    # a norm weight of ones: RMSNorm without its weight, for the calls whose
    # projection (holding the folded weight) reads a normalised input
    unit_norm: torch.Tensor = field(repr=False, default=None)

    def __post_init__(self):
        if self.unit_norm is None:
            self.unit_norm = torch.ones(self.config.hidden_size, dtype=self.embed.dtype, device=self.embed.device)

    @property
    def device(self) -> torch.device:
        return self.embed.device

    @property
    def dtype(self) -> torch.dtype:
        return self.embed.dtype

    @property
    def scaling(self) -> float:
        return self.config.head_dim ** -0.5

    def ensure_positions(self, n: int) -> None:
        if n > self.rope_cos.shape[0]:
            cos, sin = rope_tables(self.config, max(n, 2 * self.rope_cos.shape[0]))
            self.rope_cos, self.rope_sin = cos.to(self.device), sin.to(self.device)

    @classmethod
    def from_state_dict(cls, shape: LlamaShape, state: dict[str, torch.Tensor], device=None,
                        dtype: torch.dtype | None = None) -> "Llama":
        def get(name):
            w = state[name]
            if device is not None or dtype is not None:
                w = w.to(device=device or w.device, dtype=dtype or w.dtype)
            return w.contiguous()

        embed = get("model.embed_tokens.weight")
        layers = []
        for n in range(shape.num_hidden_layers):
            p = f"model.layers.{n}."
            ln1, ln2 = get(p + "input_layernorm.weight"), get(p + "post_attention_layernorm.weight")
            wqkv = torch.cat([get(p + "self_attn.q_proj.weight"), get(p + "self_attn.k_proj.weight"),
                              get(p + "self_attn.v_proj.weight")], dim=0)
            wgu = torch.cat([get(p + "mlp.gate_proj.weight"), get(p + "mlp.up_proj.weight")], dim=0)
            layers.append(Layer(ln1, fold_norm(wqkv, ln1), get(p + "self_attn.o_proj.weight"), ln2,
                                fold_norm(wgu, ln2), get(p + "mlp.down_proj.weight")))
        head = embed if shape.tie_word_embeddings else get("lm_head.weight")
        if head.is_cuda and head.dtype in (torch.bfloat16, torch.float16):
            wide = head
        else:
            wide = head.to(torch.promote_types(head.dtype, torch.float32)).contiguous()
        cos, sin = rope_tables(shape, shape.max_position_embeddings)
        return cls(shape, embed, layers, get("model.norm.weight"), head, wide, cos.to(embed.device),
                   sin.to(embed.device))

    @classmethod
    def random(cls, shape: LlamaShape, seed: int, device, dtype: torch.dtype = torch.bfloat16) -> "Llama":
        return cls.from_state_dict(shape, random_state_dict(shape, seed, device, dtype))


def rope_tables(shape: LlamaShape, n_positions: int) -> tuple[torch.Tensor, torch.Tensor]:
    """fp32 cos/sin [n_positions, head_dim/2] (CPU), computed as
    transformers' default rotary embedding does."""
    d = shape.head_dim
    inv_freq = 1.0 / (shape.rope_theta ** (torch.arange(0, d, 2, dtype=torch.int64).float() / d))
    pos = torch.arange(n_positions, dtype=torch.float32)
    angle = pos[:, None] * inv_freq[None, :]
    return angle.cos().contiguous(), angle.sin().contiguous()


def shape_from_hf_config(config) -> LlamaShape:
    """The Llama shape of a transformers config.  Architectures whose math
    this forward does not carry are refused rather than run with wrong
    logits: projection biases (Qwen2's q/k/v biases, `attention_bias`,
    `mlp_bias`), scaled RoPE (`rope_scaling` other than the default) and
    sliding-window attention."""
    head_dim = getattr(config, "head_dim", None) or config.hidden_size // config.num_attention_heads
    if config.model_type != "llama":
        raise NotImplementedError(f"the forward implements the Llama architecture; got {config.model_type} "
                                  "(Qwen2's q/k/v projection biases are not implemented)")
    if getattr(config, "attention_bias", False) or getattr(config, "mlp_bias", False):
        raise NotImplementedError("projection biases (attention_bias / mlp_bias) are not implemented")
    scaling = getattr(config, "rope_scaling", None)
    params = getattr(config, "rope_parameters", None)
    kind = None
    for source in (scaling, params):
        if isinstance(source, dict):
            kind = source.get("rope_type", source.get("type")) or kind
    if kind not in (None, "default"):
        raise NotImplementedError(f"RoPE scaling {kind!r} is not implemented (only the default rotary tables)")
    if getattr(config, "use_sliding_window", False):
        raise NotImplementedError("sliding-window attention is not implemented")
    return LlamaShape(
        vocab_size=config.vocab_size, hidden_size=config.hidden_size, num_hidden_layers=config.num_hidden_layers,
        num_attention_heads=config.num_attention_heads, num_key_value_heads=config.num_key_value_heads,
        intermediate_size=config.intermediate_size, head_dim=head_dim, rms_norm_eps=config.rms_norm_eps,
        rope_theta=float(getattr(config, "rope_theta", None) or config.rope_parameters["rope_theta"]),
        tie_word_embeddings=bool(getattr(config, "tie_word_embeddings", False)),
        max_position_embeddings=config.max_position_embeddings)


def as_llama(model, device=None) -> Llama:
    """Our Llama, or a transformers LlamaForCausalLM converted once (onto
    `device`, default the model's own) and cached on it."""
    if isinstance(model, Llama):
        return model
    cached = getattr(model, "_specdec_llama", None)
    if cached is not None and (
            (device is not None and cached.device != torch.device(device))
            or len(cached.layers) != model.config.num_hidden_layers):
        cached = None
    if cached is None:
        shape = shape_from_hf_config(model.config)
        state = {k: v.detach() for k, v in model.state_dict().items()}
        if shape.tie_word_embeddings is False and "lm_head.weight" not in state:
            shape = shape.replace(tie_word_embeddings=True)
        cached = Llama.from_state_dict(shape, state, device=device)
        model._specdec_llama = cached
    return cached
