"""Target verification pass (reference: spec/verify.py:9-30)."""
from __future__ import annotations

import torch

from cache.kv import KVCache
from lm import graphs
from lm.forward import forward
from lm.model import as_llama


def verify(target, cache: KVCache, seq_ids: list[int], contexts: list[list[int]], draft: torch.Tensor,
           temperature: float) -> torch.Tensor:
    """p [B, k+1, V] float32, in GPU memory, for accept_reject.

    Each row feeds k+1 tokens at once: the last context token, whose KV the
    target has not cached yet, followed by the k drafted ids.  The softmax
    (or one-hot, at temperature 0) after input position j is what the
    target would emit there: positions 0..k-1 judge drafts 1..k, position k
    gives the extra token emitted when every draft is kept.  The new tokens
    occupy cache positions len(context) - 1 .. len(context) + k - 1, so the
    cache must hold exactly len(context) - 1 positions on entry."""
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
