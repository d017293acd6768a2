"""Plain cached decoding: the greedy oracle of the identity checks and the
non-speculative baseline (reference contract: baselines/cached_autoregressive.py:11-90).

Both entry points run one decoder, `_decode`: a prefill forward over the
right-padded prompts (each row's last real position projected), then one
forward per step over the rows still running, each feeding its previous
token.  A row stops at eos or after max_new_tokens tokens and leaves the
batch (its cache sequence is freed there and then), so a batch does the same
work per row as single-row decoding.  Greedy steps take one argmax over the
live rows' logits (the first maximum wins: ties go to the lower id) and one
host copy; sampled steps draw per row, in row order, from `generator`.
"""
from __future__ import annotations

from collections.abc import Callable

import torch

from cache.kv import KVCache
from lm.forward import forward
from lm.sampling import next_token


def _choose(logits: torch.Tensor, temperature: float, generator: torch.Generator | None) -> list[int]:
    """Next token of every row of logits [B, V]."""
    if temperature == 0.0:
        return logits.argmax(dim=-1).tolist()
    return [next_token(row, temperature, generator) for row in logits]


def _decode(model, cache: KVCache, seq_ids: list[int], prompts: list[list[int]], max_new_tokens: int,
            temperature: float, generator: torch.Generator | None, eos_id: int | None,
            on_event: Callable[[str], None] | None) -> list[list[int]]:
    for s in seq_ids:
        cache.add(s)
    try:
        width = max(len(p) for p in prompts)
        padded = torch.tensor([p + [0] * (width - len(p)) for p in prompts], dtype=torch.int64)
        logits = forward(model, cache, seq_ids, padded, [len(p) for p in prompts], last_only=True)
        outs: dict[int, list[int]] = {s: [] for s in seq_ids}
        running = list(seq_ids) if max_new_tokens > 0 else []  # a zero budget stops after the prefill
        first = True
        while running:
            for s, token in zip(running, _choose(logits, temperature, generator)):
                outs[s].append(token)
            if first and on_event is not None:
                on_event("first_token")
            first = False
            still = []
            for s in running:
                out = outs[s]
                if out[-1] == eos_id or len(out) >= max_new_tokens:
                    cache.free(s)
                else:
                    still.append(s)
            running = still
            if running:
                step = torch.tensor([[outs[s][-1]] for s in running], dtype=torch.int64)
                logits = forward(model, cache, running, step, [1] * len(running))[:, 0]
        return [outs[s] for s in seq_ids]
    finally:
        for s in seq_ids:
            if s in cache.tables:
                cache.free(s)


@torch.no_grad()
def generate(model, cache: KVCache, prompt: list[int], max_new_tokens: int, temperature: float = 0.0,
             generator: torch.Generator | None = None, eos_id: int | None = None, seq_id: int = 0,
             on_event: Callable[[str], None] | None = None) -> list[int]:
    """Up to max_new_tokens tokens after `prompt` (ending early at eos), as
    sequence `seq_id` of `cache`, which is freed again before returning."""
    return _decode(model, cache, [seq_id], [prompt], max_new_tokens, temperature, generator, eos_id, on_event)[0]


@torch.no_grad()
def generate_batch(model, cache: KVCache, prompts: list[list[int]], max_new_tokens: int, temperature: float = 0.0,
                   generator: torch.Generator | None = None, eos_id: int | None = None,
                   on_event: Callable[[str], None] | None = None) -> list[list[int]]:
    """Every prompt decoded at once as sequences 0..B-1 of `cache`, one
    forward per step over the rows still running."""
    return _decode(model, cache, list(range(len(prompts))), prompts, max_new_tokens, temperature, generator, eos_id,
                   on_event)
