"""Target verification pass (reference: spec/verify.py:9-30)."""
from __future__ import annotations

import torch

from cache.kv import KVCache
from lm import graphs
from lm.forward import forward
from lm.model import as_llama


def verify(target, cache: KVCache, seq_ids: list[int], contexts: list[list[int]], draft: torch.Tensor,
           temperature: float) -> torch.Tensor:
    """One target forward over [context[-1], d_1, ..., d_k] per row.  Output row
    i is the target's distribution for the token after d_i (row 0: for d_1
    itself) and row k is the bonus position.  Returns p [B, k+1, V] float32.

    p stays in GPU memory: its only consumer is accept_reject, which runs
    there.  Positions run from len(context) - 1 to len(context) + k - 1, set
    by the cache's per-row past length."""
    for seq_id, ctx in zip(seq_ids, contexts):
        if cache.length(seq_id) != len(ctx) - 1:
            raise RuntimeError(f"seq {seq_id}: target cache holds {cache.length(seq_id)}, expected {len(ctx) - 1}")
    last = torch.tensor([[ctx[-1]] for ctx in contexts], dtype=torch.int64).to(cache.device, non_blocking=True)
    input_ids = torch.cat([last, draft.to(cache.device, torch.int64)], dim=1)
    b, k1 = input_ids.shape
    if not graphs.enabled():
        return forward(target, cache, seq_ids, input_ids, [k1] * b, temperature=temperature)
    llama = as_llama(target, cache.device)
    step = cache.append(seq_ids, [k1] * b)
    llama.ensure_positions(step.max_total)
    runner = graphs.get(cache, graphs.VerifyGraph, llama, b, k1, float(temperature),
                        graphs.bucket_for(step.max_total))
    # a copy: the runner's output buffer is overwritten by its next replay
    return runner.run(input_ids, step.meta).clone()
