"""The speculative round loop (reference: spec/loop.py:14-129).

Same contract and bookkeeping as the reference's `generate`: the first token
comes from the target's prefill, each round drafts k tokens, verifies them in
one target pass, keeps the accepted prefix plus the correction or bonus
token, trims to the budget and eos, and rolls both caches back so the target
cache holds all but the last context token.
"""
from __future__ import annotations

from collections.abc import Callable
from dataclasses import dataclass, field

import torch

from cache.kv import KVCache
from lm.sampling import probabilities
from spec.accept import accept_reject
from spec.draft import Drafter, run, sample
from spec.verify import verify


@dataclass
class SpecStats:
    k: int
    rounds: int = 0
    drafted: int = 0
    accepted: int = 0
    # attempts[i]: rounds that reached draft position i; accepts[i]: of those, accepted there
    attempts: list[int] = field(default_factory=list)
    accepts: list[int] = field(default_factory=list)
    # per (sequence, round): tokens emitted that round after eos/budget trimming
    emitted_per_round: list[int] = field(default_factory=list)
    # same indexing: how many of those were accepted draft tokens
    drafted_per_round: list[int] = field(default_factory=list)

    def __post_init__(self) -> None:
        self.attempts = [0] * self.k
        self.accepts = [0] * self.k

    @property
    def discarded(self) -> int:
        return self.drafted - self.accepted


@torch.no_grad()
def generate(target, cache: KVCache, drafter: Drafter, prompts: list[list[int]], max_new_tokens: int, k: int,
             temperature: float = 0.0, generator: torch.Generator | None = None, eos_id: int | None = None,
             on_event: Callable[[str], None] | None = None) -> tuple[list[list[int]], SpecStats]:
    generator = generator or torch.Generator().manual_seed(0)
    stats = SpecStats(k)
    notify = on_event or (lambda name: None)
    seq_ids = list(range(len(prompts)))
    for s in seq_ids:
        cache.add(s)
    # first token from the target prefill, as in plain decoding
    first_probs = probabilities(run(target, cache, seq_ids, prompts), temperature)
    first = sample(first_probs, generator).tolist()
    notify("first_token")
    drafter.prefill(seq_ids, prompts)
    notify("draft_prefilled")
    contexts = [list(p) + [t] for p, t in zip(prompts, first)]
    outputs = [[t] for t in first]
    active = []
    for s in seq_ids:
        if finished(outputs[s], max_new_tokens, eos_id):
            release(cache, drafter, s)
        else:
            active.append(s)

    while active:
        ctx = [contexts[s] for s in active]
        draft, q = drafter.propose(active, ctx, k, temperature, generator)
        p = verify(target, cache, active, ctx, draft, temperature)
        verdict = accept_reject(p, q, draft, generator=generator)
        stats.rounds += 1
        draft_host = draft.cpu()
        n_acc = verdict.n_accepted.tolist()
        nxt = verdict.next_token.tolist()
        survivors = []
        for row, s in enumerate(active):
            n = n_acc[row]
            record(stats, n)
            new = trim(draft_host[row, :n].tolist() + [nxt[row]], len(outputs[s]), max_new_tokens, eos_id)
            stats.emitted_per_round.append(len(new))
            stats.drafted_per_round.append(min(n, len(new)))
            before = len(contexts[s])
            contexts[s] = contexts[s] + new
            outputs[s] = outputs[s] + new
            if finished(outputs[s], max_new_tokens, eos_id):
                release(cache, drafter, s)
                continue
            # the target cache held context[:-1] plus the k+1 verified slots;
            # keeping n drafts and one correction leaves `before + n` cached
            cache.truncate(s, before + n)
            drafter.rollback(s, before + n)
            survivors.append(s)
        active = survivors
        if stats.rounds == 1:
            notify("first_round")
    return outputs, stats


def record(stats: SpecStats, n: int) -> None:
    stats.drafted += stats.k
    stats.accepted += n
    for i in range(min(n + 1, stats.k)):
        stats.attempts[i] += 1
    for i in range(n):
        stats.accepts[i] += 1


def trim(new: list[int], have: int, max_new_tokens: int, eos_id: int | None) -> list[int]:
    new = new[: max_new_tokens - have]
    if eos_id is not None and eos_id in new:
        new = new[: new.index(eos_id) + 1]
    return new


def finished(output: list[int], max_new_tokens: int, eos_id: int | None) -> bool:
    return len(output) >= max_new_tokens or (eos_id is not None and output[-1] == eos_id)


def release(cache: KVCache, drafter: Drafter, seq_id: int) -> None:
    cache.free(seq_id)
    drafter.release(seq_id)
