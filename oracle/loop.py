"""Oracle of spec/loop.py and baselines/cached_autoregressive.py (test
infrastructure, see oracle/__init__.py)."""
from dataclasses import dataclass, field

import torch

from oracle.accept import accept_reject
from oracle.draft import run, sample, verify
from oracle.forward import forward
from oracle.sampling import next_token, probabilities


@dataclass
class SpecStats:
    """spec/loop.py:14-35"""
    k: int
    rounds: int = 0
    drafted: int = 0
    accepted: int = 0
    attempts: list = field(default_factory=list)
    accepts: list = field(default_factory=list)
    emitted_per_round: list = field(default_factory=list)
    drafted_per_round: list = field(default_factory=list)

    def __post_init__(self):
        self.attempts = [0] * self.k
        self.accepts = [0] * self.k


@torch.no_grad()
def generate(target, cache, drafter, prompts, max_new_tokens, k, temperature=0.0, generator=None, eos_id=None):
    """spec/loop.py:38-104"""
    generator = generator or torch.Generator().manual_seed(0)
    stats = SpecStats(k)
    seq_ids = list(range(len(prompts)))
    for s in seq_ids:
        cache.add(s)
    first = sample(probabilities(run(target, cache, seq_ids, prompts), temperature), generator).tolist()
    drafter.prefill(seq_ids, prompts)
    contexts = [p + [t] for p, t in zip(prompts, first)]
    outputs = [[t] for t in first]
    active = [s for s in seq_ids if not _finished(outputs[s], max_new_tokens, eos_id)]
    for s in seq_ids:
        if s not in active:
            cache.free(s)
            drafter.release(s)
    while active:
        ctx = [contexts[s] for s in active]
        draft, q = drafter.propose(active, ctx, k, temperature, generator)
        p = verify(target, cache, active, ctx, draft, temperature)
        verdict = accept_reject(p, q, draft, generator=generator)
        stats.rounds += 1
        still = []
        for row, s in enumerate(active):
            n = int(verdict.n_accepted[row])
            stats.drafted += k
            stats.accepted += n
            for i in range(min(n + 1, k)):
                stats.attempts[i] += 1
            for i in range(n):
                stats.accepts[i] += 1
            new = draft[row, :n].tolist() + [int(verdict.next_token[row])]
            new = new[: max_new_tokens - len(outputs[s])]
            if eos_id is not None and eos_id in new:
                new = new[: new.index(eos_id) + 1]
            stats.emitted_per_round.append(len(new))
            stats.drafted_per_round.append(min(n, len(new)))
            before = len(contexts[s])
            contexts[s] = contexts[s] + new
            outputs[s] = outputs[s] + new
            if _finished(outputs[s], max_new_tokens, eos_id):
                cache.free(s)
                drafter.release(s)
                continue
            cache.truncate(s, before + n)
            drafter.rollback(s, before + n)
            still.append(s)
        active = still
    return outputs, stats


def _finished(output, max_new_tokens, eos_id):
    return len(output) >= max_new_tokens or (eos_id is not None and output[-1] == eos_id)


@torch.no_grad()
def greedy(model, cache, prompt, max_new_tokens, eos_id=None, seq_id=0):
    """baselines/cached_autoregressive.py:11-39 at temperature 0"""
    cache.add(seq_id)
    try:
        logits = forward(model, cache, [seq_id], torch.tensor([prompt]), [len(prompt)], last_only=True)[0]
        out = []
        for _ in range(max_new_tokens):
            token = next_token(logits, 0.0, None)
            out.append(token)
            if token == eos_id or len(out) == max_new_tokens:
                break
            logits = forward(model, cache, [seq_id], torch.tensor([[token]]), [1])[0, 0]
        return out
    finally:
        cache.free(seq_id)
