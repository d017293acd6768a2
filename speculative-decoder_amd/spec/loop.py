"""Round driver of speculative decoding (reference contract: spec/loop.py:14-129).

What a caller of the reference's `generate` relies on, and what this driver keeps:

* events, in order: "first_token" once the target prefill's token is sampled,
  "draft_prefilled" after the drafter's prefill, "first_round" after the first
  round is settled;
* draws from `generator`, in order: one uniform per row for the first token
  (spec/draft.py:27-29), then per round whatever the drafter draws, then
  accept_reject's u_accept [B, k] and u_residual [B] (spec/accept.py:60-63);
* `SpecStats` fields and their per-(sequence, round) bookkeeping;
* caches: a round that keeps n drafts leaves the target cache at the
  pre-round context length + n, i.e. the new context minus its last token,
  and the drafter is rolled back to the same length; a finished sequence is
  released from both, at once;
* `verify` is read from this module's globals at call time (tests patch
  spec.loop.verify).

How it is organised: every prompt becomes a `_Request` holding its context
and output.  A round proposes, verifies and decides for all live requests,
brings the verdict and the draft to the host in one copy, then settles
in two phases: `_plan` works out each request's kept tokens, statistics and
cache action on the host alone; `_apply` carries the actions out in request
order (the cache's rollbacks are queued and reach the device with the next
append as one block-plan launch).
"""
from __future__ import annotations

from collections.abc import Callable
from dataclasses import dataclass, field

import torch

from cache.kv import KVCache
from lm.sampling import probabilities
from spec.accept import accept_reject, host_draft
from spec.draft import Drafter, run, sample
from spec.verify import verify


@dataclass
class SpecStats:
    """Acceptance bookkeeping of one `generate` call.

    attempts[i] counts the (sequence, round) pairs that tested draft position
    i -- they accepted every earlier position -- and accepts[i] those that
    accepted it too.  emitted_per_round and drafted_per_round hold one entry
    per (sequence, round), in settle order: the tokens the round emitted after
    the budget/eos cut, and how many of them were accepted draft tokens (the
    rest is the target's correction or bonus token)."""

    k: int
    rounds: int = 0
    drafted: int = 0
    accepted: int = 0
    attempts: list[int] = field(default_factory=list)
    accepts: list[int] = field(default_factory=list)
    emitted_per_round: list[int] = field(default_factory=list)
    drafted_per_round: list[int] = field(default_factory=list)

    def __post_init__(self) -> None:
        self.attempts = [0] * self.k
        self.accepts = [0] * self.k

    @property
    def discarded(self) -> int:
        return self.drafted - self.accepted

    def tally(self, n: int, emitted: int) -> None:
        """One (sequence, round) that accepted n of its k drafts and emitted
        `emitted` tokens after the cut.  Positions 0..n were tested (all k
        when every draft was accepted)."""
        self.drafted += self.k
        self.accepted += n
        for i in range(min(n + 1, self.k)):
            self.attempts[i] += 1
            self.accepts[i] += i < n
        self.emitted_per_round.append(emitted)
        self.drafted_per_round.append(min(n, emitted))


@dataclass
class _Request:
    seq_id: int
    context: list[int]
    output: list[int] = field(default_factory=list)

    def extend(self, tokens: list[int]) -> None:
        # in place: a drafter that keeps a device copy of the context (the
        # n-gram drafter) sees the same list grow and uploads only the new
        # tokens, a cost independent of the context's length
        self.context.extend(tokens)
        self.output.extend(tokens)

    def done(self, max_new_tokens: int, eos_id: int | None) -> bool:
        return len(self.output) >= max_new_tokens or (eos_id is not None and self.output[-1] == eos_id)


def _cut(tokens: list[int], room: int, eos_id: int | None) -> list[int]:
    """The tokens a round may emit: at most `room` (the budget left), and
    nothing after the first eos."""
    kept = tokens[:room]
    if eos_id is not None and eos_id in kept:
        kept = kept[: kept.index(eos_id) + 1]
    return kept


@dataclass(frozen=True)
class _Action:
    """What one settled request does to the caches: release it, or keep
    `keep` positions (the context minus its last token)."""

    seq_id: int
    release: bool
    keep: int


def _plan(live: list[_Request], n_accepted: list[int], drafts: list[list[int]], corrections: list[int],
          stats: SpecStats, max_new_tokens: int, eos_id: int | None) -> tuple[list[_Request], list[_Action]]:
    """Host half of a round's settlement: kept tokens, statistics, and the
    cache action of every live request, in request order."""
    survivors, actions = [], []
    for req, n, drafted, correction in zip(live, n_accepted, drafts, corrections):
        kept = _cut(drafted[:n] + [correction], max_new_tokens - len(req.output), eos_id)
        stats.tally(n, len(kept))
        before = len(req.context)
        req.extend(kept)
        # the target cache held context[:-1] plus the k + 1 verified slots;
        # keeping n drafts and one correction leaves before + n cached
        finished = req.done(max_new_tokens, eos_id)
        actions.append(_Action(req.seq_id, finished, before + n))
        if not finished:
            survivors.append(req)
    return survivors, actions


def _apply(actions: list[_Action], cache: KVCache, drafter: Drafter) -> None:
    for act in actions:
        if act.release:
            _release(cache, drafter, act.seq_id)
        else:
            cache.truncate(act.seq_id, act.keep)
            drafter.rollback(act.seq_id, act.keep)


def _release(cache: KVCache, drafter: Drafter, seq_id: int) -> None:
    cache.free(seq_id)
    drafter.release(seq_id)


@torch.no_grad()
def generate(target, cache: KVCache, drafter: Drafter, prompts: list[list[int]], max_new_tokens: int, k: int,
             temperature: float = 0.0, generator: torch.Generator | None = None, eos_id: int | None = None,
             on_event: Callable[[str], None] | None = None) -> tuple[list[list[int]], SpecStats]:
    """Speculative decoding of `prompts` with target `target` and `drafter`
    proposing k tokens per round; returns each prompt's new tokens and the
    acceptance statistics.  Temperature 0 reproduces plain greedy decoding of
    the target; above 0 every token is distributed as the target's softmax."""
    gen = generator if generator is not None else torch.Generator().manual_seed(0)
    event = on_event if on_event is not None else (lambda name: None)
    stats = SpecStats(k)
    requests = [_Request(i, list(p)) for i, p in enumerate(prompts)]
    seq_ids = [r.seq_id for r in requests]
    for s in seq_ids:
        cache.add(s)
    firsts = sample(probabilities(run(target, cache, seq_ids, prompts), temperature), gen).tolist()
    event("first_token")
    drafter.prefill(seq_ids, [r.context for r in requests])  # the prompts, as the lists that will grow
    event("draft_prefilled")
    live = []
    for req, token in zip(requests, firsts):
        req.extend([token])
        if req.done(max_new_tokens, eos_id):
            _release(cache, drafter, req.seq_id)
        else:
            live.append(req)

    while live:
        ids = [r.seq_id for r in live]
        contexts = [r.context for r in live]
        draft, q = drafter.propose(ids, contexts, k, temperature, gen)
        p = verify(target, cache, ids, contexts, draft, temperature)
        verdict = accept_reject(p, q, draft, generator=gen)
        stats.rounds += 1
        drafted = host_draft(verdict)
        if drafted is None:
            drafted = draft
        live, actions = _plan(live, verdict.n_accepted.tolist(), drafted.tolist(), verdict.next_token.tolist(), stats,
                              max_new_tokens, eos_id)
        _apply(actions, cache, drafter)
        if stats.rounds == 1:
            event("first_round")
    return [r.output for r in requests], stats
