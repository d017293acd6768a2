"""Cached Llama forward over the paged cache (reference: lm/forward.py:21-84).

Per layer: RMSNorm, one fused QKV GEMM (torch/hipBLASLt), the fused RoPE +
paged append kernel, the paged verify-attention kernel reading K/V blocks in
place (no gather copy, no materialised mask), o_proj, RMSNorm and the SwiGLU
MLP as two GEMMs.  The output projection runs in at least fp32, as in the
reference (lm/forward.py:71-84).
"""
from __future__ import annotations

import torch
import torch.nn.functional as F

from cache.kv import KVCache
from lm.model import Llama, as_llama
from specdec import ops


def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    """transformers' LlamaRMSNorm: normalise in fp32, cast back, then scale."""
    h = x.float()
    h = h * torch.rsqrt(h.pow(2).mean(-1, keepdim=True) + eps)
    return weight * h.to(x.dtype)


@torch.no_grad()
def forward(model, cache: KVCache, seq_ids: list[int], input_ids: torch.Tensor, n_new: list[int],
            last_only: bool = False) -> torch.Tensor:
    """Run `input_ids` [B, T] (right-padded; row b has n_new[b] real tokens)
    through the model, appending to each sequence's cache.  Returns logits
    [B, T, V]; rows past n_new[b] are padding.  With `last_only`, only each
    row's last real token is projected and the result is [B, V].

    The same call serves prefill (T = prompt length), decode (T = 1) and
    speculative verification (T = k + 1)."""
    llama = as_llama(model, cache.device)
    cfg = llama.config
    step = cache.append(seq_ids, n_new)
    ids = input_ids.to(cache.device, non_blocking=True)
    b, t = ids.shape
    llama.ensure_positions(step.max_total)
    h, hk, d = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim
    hidden = F.embedding(ids, llama.embed)
    attn = torch.empty(b, t, h * d, dtype=hidden.dtype, device=hidden.device)
    tables = cache.table_tensor
    inter = cfg.intermediate_size
    for i, layer in enumerate(llama.layers):
        x = rms_norm(hidden, layer.ln1, cfg.rms_norm_eps)
        qkv = F.linear(x, layer.wqkv)
        ops.rope_append(qkv, h, hk, d, llama.rope_cos, llama.rope_sin, step.meta, b, t, tables,
                        cache.block_size, cache.k[i], cache.v[i])
        ops.paged_attention(qkv, qkv.stride(1), cache.k[i], cache.v[i], tables, step.meta, b, t, h, hk, d,
                            cache.block_size, llama.scaling, step.max_total, attn, attn.stride(1))
        hidden = hidden + F.linear(attn, layer.wo)
        x = rms_norm(hidden, layer.ln2, cfg.rms_norm_eps)
        gu = F.linear(x, layer.wgu)
        hidden = hidden + F.linear(F.silu(gu[..., :inter]) * gu[..., inter:], layer.wd)
    if last_only:
        last = torch.tensor([n - 1 for n in n_new], device=hidden.device)
        hidden = hidden[torch.arange(b, device=hidden.device), last]
    return logits(llama, rms_norm(hidden, llama.norm, cfg.rms_norm_eps))


def logits(model, hidden: torch.Tensor) -> torch.Tensor:
    """The output projection in at least fp32: in bf16 near-tied candidates
    round to the same logit and argmax would break the tie by whichever
    rounding a (k+1)-token verify and a 1-token decode produced."""
    llama = as_llama(model)
    wide = llama.head_wide
    return F.linear(hidden.to(wide.dtype), wide)


__all__ = ["forward", "logits", "rms_norm", "Llama"]
