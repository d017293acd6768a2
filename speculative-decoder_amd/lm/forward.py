"""Cached Llama forward over the paged cache (reference: lm/forward.py:21-84).

A forward is split in two:
  * host part: `cache.append` decides block growth (one block-plan launch)
    and uploads the per-row metadata (table row, past length, new tokens);
  * device part, `forward_core`: eight launches per layer (nine when the
    attention needs its split combine) -- fused residual add + RMSNorm, one
    fused QKV GEMM (torch/hipBLASLt), the paged verify-attention kernel that
    also applies RoPE and appends the new K/V to the paged pools and reads
    K/V blocks in place (no gather copy, no materialised mask), o_proj, add
    + RMSNorm, the gate/up GEMM, SiLU*up, the down GEMM -- then the fp32
    output projection (lm/forward.py:71-84).
The device part reads everything it needs from device memory, so a fixed
(batch, width) shape can be captured once in a HIP graph and replayed
(lm/graphs.py).
"""
from __future__ import annotations

import torch
import torch.nn.functional as F

from cache.kv import KVCache
from lm.model import Llama, as_llama
from specdec import ops


def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    """transformers' LlamaRMSNorm on the GPU (fused kernel)."""
    x = x.contiguous()
    out = torch.empty_like(x)
    return ops.add_rmsnorm(x.clone(), None, weight, out, eps)


def _project(x: torch.Tensor, w: torch.Tensor, gemv: bool) -> torch.Tensor:
    """x @ w.T on torch: a matrix-vector product when asked for and x is a
    single row (about a microsecond less per call at decode sizes), else the
    GEMM.  The two may round differently, so a model uses one of them for
    every call whose bits must agree."""
    if gemv and x.numel() == x.shape[-1]:
        return torch.mv(w, x.reshape(-1)).view(*x.shape[:-1], w.shape[0])
    return F.linear(x, w)


def forward_core(llama: Llama, cache: KVCache, meta: torch.Tensor, ids: torch.Tensor, max_kv_len: int,
                 last: torch.Tensor | None = None, workspace: ops.AttentionWorkspace | None = None,
                 split_tokens: int = 0) -> torch.Tensor:
    """Device-only forward of ids [B, T] whose rows were appended with `meta`
    (int32 [3, B] on the device).  `max_kv_len` bounds every row's cached
    length after the append; `last` (int64 [B]) selects one row per batch
    entry before the output projection.  `split_tokens` is the attention
    split (0: the fixed default whose results do not depend on the other
    queries of the call; nonzero marks a latency call -- the draft -- whose
    bits need not match other calls, which also lets single-row projections
    run as matrix-vector products)."""
    cfg = llama.config
    gemv = split_tokens != 0
    b, t = ids.shape
    h, hk, d, inter, eps = (cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim, cfg.intermediate_size,
                            cfg.rms_norm_eps)
    tables = cache.table_tensor
    layers = llama.layers
    hidden = F.embedding(ids, llama.embed)
    x = torch.empty_like(hidden)
    ops.add_rmsnorm(hidden, None, layers[0].ln1, x, eps)
    attn = torch.empty(b, t, h * d, dtype=hidden.dtype, device=hidden.device)
    act = torch.empty(b, t, inter, dtype=hidden.dtype, device=hidden.device)
    for i, layer in enumerate(layers):
        qkv = _project(x, layer.wqkv, gemv)
        ops.rope_paged_attention(qkv, llama.rope_cos, llama.rope_sin, cache.k[i], cache.v[i], tables, meta, b, t, h,
                                 hk, d, cache.block_size, llama.scaling, max_kv_len, attn, attn.stride(1), workspace,
                                 split_tokens)
        ops.add_rmsnorm(hidden, _project(attn, layer.wo, gemv), layer.ln2, x, eps)
        ops.silu_mul(_project(x, layer.wgu, gemv), act)
        nxt = layers[i + 1].ln1 if i + 1 < len(layers) else llama.norm
        ops.add_rmsnorm(hidden, _project(act, layer.wd, gemv), nxt, x, eps)
    if last is not None:
        x = x[torch.arange(b, device=x.device), last]
    return logits(llama, x)


@torch.no_grad()
def forward(model, cache: KVCache, seq_ids: list[int], input_ids: torch.Tensor, n_new: list[int],
            last_only: bool = False, latency_split: bool = False) -> torch.Tensor:
    """Run `input_ids` [B, T] (right-padded; row b has n_new[b] real tokens)
    through the model, appending to each sequence's cache.  Returns logits
    [B, T, V]; rows past n_new[b] are padding.  With `last_only`, only each
    row's last real token is projected and the result is [B, V].

    The same call serves prefill (T = prompt length), decode (T = 1) and
    speculative verification (T = k + 1).  `latency_split` lets attention
    pick a split for latency (the draft) instead of the fixed default."""
    llama = as_llama(model, cache.device)
    step = cache.append(seq_ids, n_new)
    ids = input_ids.to(cache.device, non_blocking=True)
    llama.ensure_positions(step.max_total)
    last = None
    if last_only:
        last = torch.tensor([n - 1 for n in n_new], dtype=torch.int64).pin_memory().to(cache.device,
                                                                                          non_blocking=True)
    cfg = llama.config
    split = (ops.latency_split(ids.shape[0], ids.shape[1], cfg.num_attention_heads, cfg.num_key_value_heads,
                               step.max_total) if latency_split else 0)
    return forward_core(llama, cache, step.meta, ids, step.max_total, last, split_tokens=split)


def logits(model, hidden: torch.Tensor) -> torch.Tensor:
    """The output projection with fp32 accumulation and fp32 logits: in bf16
    near-tied candidates round to the same logit and argmax would break the
    tie by whichever rounding a (k+1)-token verify and a 1-token decode
    produced.  The reference multiplies by an fp32 copy of the head
    (lm/forward.py:71-84); bf16 weights are read here as stored, half the
    bytes, and since the product of two bf16 values is exact in fp32 the
    arithmetic is the fp32 head's up to the GEMM's summation order."""
    llama = as_llama(model)
    w = llama.head_wide
    if w.dtype not in (torch.bfloat16, torch.float16):
        return F.linear(hidden.to(w.dtype), w)
    flat = hidden.reshape(-1, hidden.shape[-1]).to(w.dtype)
    return torch.mm(flat, w.t(), out_dtype=torch.float32).view(*hidden.shape[:-1], w.shape[0])
