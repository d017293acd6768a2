"""Cached Llama forward over the paged cache (reference: lm/forward.py:21-84).

A forward is split in two:
  * host part: `cache.append` decides block growth (one block-plan launch)
    and uploads the per-row metadata (table row, past length, new tokens);
  * device part, `forward_core`: five launches per layer for decode,
    verification and draft steps (six when the attention needs its split
    combine):
      - the fused QKV projection (specdec_linear at decode sizes, else
        torch/hipBLASLt) of the unnormalised residual stream;
      - the paged attention kernel, which finishes the input RMSNorm (each
        token's q/k/v scaled by its row's rsqrt(mean(x^2) + eps)), applies
        RoPE, appends the new K/V to the paged pools and reads K/V blocks in
        place (no gather copy, no materialised mask) -- for a draft step,
        as split partials over up to 16 CUs per kv head;
      - o_proj accumulated into the residual stream by the projection itself
        (folding the draft step's partials first);
      - gate/up of the unnormalised stream with the post-attention norm and
        SiLU*up in its epilogue (specdec_linear_silu; a separate kernel
        after a torch GEMM for wider calls);
      - the down projection, again accumulated into the stream;
    then the final norm and the fp32 output projection (lm/forward.py:71-84).
    The norm weights live in the projections' columns (lm/model.py:Layer).
    Prefill (more than 16 new tokens) and fp32 models normalise in a kernel
    of their own instead, without the weight.
The device part reads everything it needs from device memory, so a fixed
(batch, width) shape can be captured once in a HIP graph and replayed
(lm/graphs.py).
"""
from __future__ import annotations

import os

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


# bf16 projections of at most this many rows run on specdec_linear (one
# pass over the weight with every load in flight; a row's bits do not
# depend on the other rows), reading the weight's tiled copy where the
# layer has one (any inner size up to 8192) and the row-major weight up to
# LINEAR_K; more rows (prompts) run on torch's GEMM.  SPECDEC_TORCH_PROJECTIONS=1
# (or LINEAR_KERNEL = False before a model's graphs are captured) keeps
# every projection on torch.
LINEAR_ROWS, LINEAR_K = 16, 2048
LINEAR_KERNEL = os.environ.get("SPECDEC_TORCH_PROJECTIONS", "0") != "1"


def _linear_weight(x: torch.Tensor, w: torch.Tensor, wt: torch.Tensor | None = None) -> torch.Tensor | None:
    """The weight specdec_linear reads for x @ w.T (w's tiled copy `wt` when
    there is one, else w), or None when the call runs on torch.  Both forms
    give the same bits."""
    k = w.shape[-1]
    if not LINEAR_KERNEL or x.numel() > LINEAR_ROWS * k:
        return None
    if wt is not None and ops.linear_fits(x, wt):
        return wt
    if k <= LINEAR_K and ops.linear_fits(x, w):
        return w
    return None


def _project(x: torch.Tensor, w: torch.Tensor, gemv: bool, wt: torch.Tensor | None = None) -> torch.Tensor:
    """x @ w.T: specdec_linear for small bf16 calls; else on torch, a
    matrix-vector product when asked for and x is a single row (about a
    microsecond less per call at decode sizes), else the GEMM.  torch's two
    may round differently, so a model uses one of them for every call whose
    bits must agree."""
    lw = _linear_weight(x, w, wt)
    if lw is not None:
        return ops.linear(x, lw)
    if gemv and x.numel() == x.shape[-1]:
        return torch.mv(w, x.reshape(-1)).view(*x.shape[:-1], w.shape[0])
    return F.linear(x, w)


def _project_add(hidden: torch.Tensor, x: torch.Tensor, w: torch.Tensor, gemv: bool,
                 wt: torch.Tensor | None = None) -> None:
    """hidden += x @ w.T inside the projection (specdec_linear's accumulate,
    or torch's GEMM with beta = 1, in place), rounded once: a residual add
    without a kernel of its own.
    A 5-row call's rows have the bits of the same rows projected alone, as
    with `_project`."""
    n, k = w.shape
    lw = _linear_weight(x, w, wt)
    if lw is not None:
        ops.linear(x, lw, out=hidden.view(-1, n), accumulate=True)
    elif gemv and x.numel() == k:
        hidden.view(n).addmv_(w, x.reshape(k))
    else:
        hidden.view(-1, n).addmm_(x.reshape(-1, k), w.t())


def forward_core(llama: Llama, cache: KVCache, meta: torch.Tensor, ids: torch.Tensor, max_kv_len: int,
                 last: torch.Tensor | None = None, workspace: ops.AttentionWorkspace | None = None,
                 split_tokens: int = 0, temperature: float | None = None, out: torch.Tensor | None = None,
                 index_out: torch.Tensor | None = None) -> torch.Tensor:
    """Device-only forward of ids [B, T] whose rows were appended with `meta`
    (int32 [3, B] on the device).  `max_kv_len` bounds every row's cached
    length after the append; `last` (int64 [B]) selects one row per batch
    entry before the output projection.  `split_tokens` is the attention
    split (0: the fixed default whose results do not depend on the other
    queries of the call; nonzero marks a latency call -- the draft -- whose
    bits need not match other calls, which also lets single-row projections
    run as matrix-vector products).  With a `temperature` the result is the
    probabilities of the logits instead (`out`, `index_out` as in
    `probabilities`)."""
    cfg = llama.config
    gemv = split_tokens != 0
    b, t = ids.shape
    h, hk, d, inter, eps = (cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim, cfg.intermediate_size,
                            cfg.rms_norm_eps)
    tables = cache.table_tensor
    layers = llama.layers
    hidden = F.embedding(ids, llama.embed)
    x = torch.empty_like(hidden)
    # the attention finishes the input norm for decode-sized calls; else a
    # weightless norm kernel writes x and the projection reads that
    in_attn = ops.norm_in_attention(hidden.dtype, cache.block_size, t)
    if not in_attn:
        ops.add_rmsnorm(hidden, None, llama.unit_norm, x, eps)
    attn = torch.empty(b, t, h * d, dtype=hidden.dtype, device=hidden.device)
    act = torch.empty(b, t, inter, dtype=hidden.dtype, device=hidden.device)
    # a draft step's attention spread over a CU per 64 keys of each kv head
    # (4 to 16), its partials folded by the o_proj launch
    parts = None
    if (in_attn and _linear_weight(attn, layers[0].wo, layers[0].wo_t) is not None and
            ops.decode_parts_fit(hidden.dtype, b, t, h, hk, d, cache.block_size, max_kv_len, split_tokens)):
        parts = ops.decode_parts_buffer(b, h, hidden.device, ops.decode_parts_count(max_kv_len))
    for i, layer in enumerate(layers):
        qkv = _project(hidden if in_attn else x, layer.wqkv, gemv, layer.wqkv_t)
        if parts is not None:
            ops.rope_paged_attention_parts(qkv, llama.rope_cos, llama.rope_sin, cache.k[i], cache.v[i], tables, meta,
                                           b, h, hk, d, cache.block_size, llama.scaling, max_kv_len, parts,
                                           norm_of=hidden, eps=eps)
            ops.linear_attn_parts(parts, b, h, _linear_weight(attn, layer.wo, layer.wo_t), hidden.view(b, -1),
                                  accumulate=True)
        else:
            ops.rope_paged_attention(qkv, llama.rope_cos, llama.rope_sin, cache.k[i], cache.v[i], tables, meta, b, t,
                                     h, hk, d, cache.block_size, llama.scaling, max_kv_len, attn, attn.stride(1),
                                     workspace, split_tokens, norm_of=hidden if in_attn else None, eps=eps)
            _project_add(hidden, attn, layer.wo, gemv, layer.wo_t)
        gw = _linear_weight(hidden, layer.wgu, layer.wgu_t)
        if gw is not None:  # gate/up and the MLP's norm + activation in one launch
            ops.linear_silu(hidden, gw, hidden, act, eps)
        else:
            ops.rms_silu_mul(_project(hidden, layer.wgu, gemv), hidden, act, eps)
        if i + 1 == len(layers):
            ops.add_rmsnorm(hidden, _project(act, layer.wd, gemv, layer.wd_t), llama.norm, x, eps)
        elif in_attn:
            _project_add(hidden, act, layer.wd, gemv, layer.wd_t)
        else:
            ops.add_rmsnorm(hidden, _project(act, layer.wd, gemv, layer.wd_t), llama.unit_norm, x, eps)
    if last is not None:
        # last is in [0, t): with one token per row it selects that token, a view
        x = x[:, 0] if t == 1 else x[torch.arange(b, device=x.device), last]
    if temperature is None:
        return logits(llama, x)
    return probabilities(llama, x, temperature, out, index_out)


@torch.no_grad()
def forward(model, cache: KVCache, seq_ids: list[int], input_ids: torch.Tensor, n_new: list[int],
            last_only: bool = False, latency_split: bool = False, temperature: float | None = None) -> torch.Tensor:
    """Run `input_ids` [B, T] (right-padded; row b has n_new[b] real tokens)
    through the model, appending to each sequence's cache.  Returns logits
    [B, T, V]; rows past n_new[b] are padding.  With `last_only`, only each
    row's last real token is projected and the result is [B, V].

    The same call serves prefill (T = prompt length), decode (T = 1) and
    speculative verification (T = k + 1).  `latency_split` lets attention
    pick a split for latency (the draft) instead of the fixed default.  With
    a `temperature` the probabilities of those logits are returned instead
    (the head and the softmax in one launch where it applies)."""
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
    return forward_core(llama, cache, step.meta, ids, step.max_total, last, split_tokens=split,
                        temperature=temperature)


def logits(model, hidden: torch.Tensor) -> torch.Tensor:
    """The output projection with fp32 accumulation and fp32 logits: in bf16
    near-tied candidates round to the same logit and argmax would break the
    tie by whichever rounding a (k+1)-token verify and a 1-token decode
    produced.  The reference multiplies by an fp32 copy of the head
    (lm/forward.py:71-84); a bf16 head is read here as stored, half the
    bytes, by the head kernel: bf16 products are exact in fp32, and the
    kernel accumulates them in one fixed order for every row, so a row's
    logits have the same bits whatever other rows share the call."""
    llama = as_llama(model)
    w = llama.head_wide
    if w.dtype == torch.bfloat16 and w.shape[1] % 32 == 0 and w.shape[1] <= 2048:
        return ops.head_logits(hidden.to(w.dtype), w)
    if w.dtype not in (torch.bfloat16, torch.float16):
        return F.linear(hidden.to(w.dtype), w)
    flat = hidden.reshape(-1, hidden.shape[-1]).to(w.dtype)
    return torch.mm(flat, w.t(), out_dtype=torch.float32).view(*hidden.shape[:-1], w.shape[0])


def probabilities(model, hidden: torch.Tensor, temperature: float, out: torch.Tensor | None = None,
                  index_out: torch.Tensor | None = None) -> torch.Tensor:
    """lm/sampling.py:13-18 applied to `logits(model, hidden)`: the head and
    the softmax / argmax in one launch for a bf16 head and a few rows (where
    it is no slower than the pair; the same logits bits, so the same
    argmax), else the logits and then the softmax kernel."""
    llama = as_llama(model)
    w = llama.head_wide
    rows = hidden.numel() // hidden.shape[-1]
    if hidden.dtype == torch.bfloat16 and ops.head_fused(w, rows, fastest=True):
        return ops.head_probabilities(hidden, w, temperature, out=out, index_out=index_out)
    return ops.probabilities(logits(llama, hidden), temperature, out=out, index_out=index_out)
