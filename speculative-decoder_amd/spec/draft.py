"""Drafters (reference: spec/draft.py).

ModelDraft keeps the whole k-step draft loop on the GPU: each step's
probabilities come from the output head fused with the softmax (the token
itself from the same launch at temperature 0), its token from the inverse-CDF
kernel with a uniform drawn from the caller's generator (the reference's
stream and order, spec/draft.py:27-29), and the sampled ids feed the next
step's forward directly, with no host round trip between steps.
"""
from __future__ import annotations

from typing import Protocol

import torch

from cache.kv import KVCache
from lm import graphs
from lm.forward import forward
from lm.model import as_llama
from spec.accept import sample_inverse_cdf


class Drafter(Protocol):
    def prefill(self, seq_ids: list[int], prompts: list[list[int]]) -> None: ...

    def propose(self, seq_ids: list[int], contexts: list[list[int]], k: int, temperature: float,
                generator: torch.Generator) -> tuple[torch.Tensor, torch.Tensor]:
        """Returns draft [B, k] and q [B, k, V]: the distributions the draft
        tokens were actually sampled from.  Accept-reject is exact only
        against those."""
        ...

    def rollback(self, seq_id: int, keep: int) -> None: ...

    def release(self, seq_id: int) -> None: ...


def sample(probs: torch.Tensor, generator: torch.Generator) -> torch.Tensor:
    """One inverse-CDF draw per row of probs [B, V] with a uniform from
    `generator` (drawn on the generator's device, in probs' dtype)."""
    dev = generator.device if generator is not None else torch.device("cpu")
    u = torch.rand(probs.shape[0], generator=generator, dtype=probs.dtype, device=dev)
    return sample_inverse_cdf(probs, u)


class ModelDraft:
    """k sequential draft forwards per round (spec/draft.py:32-62).  By
    default the draft computes for latency: single-row projections as
    matrix-vector products and an attention split chosen for speed, whose
    bits need not match the target's verify.  With exact=True it computes as
    the verify and plain decoding do (same GEMMs, the fixed split), so a
    draft that is the target itself proposes exactly the target's greedy
    tokens."""

    def __init__(self, model, cache: KVCache, exact: bool = False) -> None:
        self.model = model
        self.cache = cache
        self.exact = exact

    def prefill(self, seq_ids: list[int], prompts: list[list[int]]) -> None:
        for seq_id in seq_ids:
            self.cache.add(seq_id)
        run(self.model, self.cache, seq_ids, prompts)

    def propose(self, seq_ids: list[int], contexts: list[list[int]], k: int, temperature: float,
                generator: torch.Generator) -> tuple[torch.Tensor, torch.Tensor]:
        # whatever part of the context the draft has not cached (its last
        # token, plus the final draft of a fully accepted round, whose KV was
        # never computed) goes into the first step as one right-padded chunk
        pending: list[list[int]] | torch.Tensor = [ctx[self.cache.length(s):] for s, ctx in zip(seq_ids, contexts)]
        if graphs.enabled() and k > 0:
            return self._propose_graphs(seq_ids, pending, k, temperature, generator)
        tokens, qs = [], []
        for _ in range(k):
            q = run(self.model, self.cache, seq_ids, pending, latency_split=not self.exact, temperature=temperature)
            token = sample(q, generator)
            tokens.append(token)
            qs.append(q)
            pending = token[:, None]
        return torch.stack(tokens, dim=1), torch.stack(qs, dim=1)

    def _propose_graphs(self, seq_ids, pending, k, temperature, generator):
        """The same k steps as one block plan + one metadata upload, then two
        graph replays: the first step (right-padded pending tokens) and the
        chain of k-1 one-token steps, tokens staying on the device."""
        cache = self.cache
        b = len(seq_ids)
        llama = as_llama(self.model, cache.device)
        n_first = [len(p) for p in pending]
        width = max(n_first)
        metas, steps = cache.append_steps(seq_ids, [n_first] + [[1] * b] * (k - 1))
        max_total = steps[-1].max_total
        llama.ensure_positions(max_total)
        bucket = graphs.bucket_for(max_total)
        # the reference draws one uniform per row per step, in step order
        dev = generator.device if generator is not None else torch.device("cpu")
        u = torch.stack([torch.rand(b, generator=generator, dtype=torch.float32, device=dev) for _ in range(k)])
        u = u.to(cache.device, non_blocking=True)
        ids = torch.tensor([p + [0] * (width - len(p)) for p in pending], dtype=torch.int64)
        latency = not self.exact
        first = graphs.get(cache, graphs.DraftStepGraph, llama, b, width, float(temperature), bucket, latency)
        q0, t0 = first.run(ids, metas[0], u[0])
        if k == 1:
            return t0.clone().view(b, 1), q0.clone().view(b, 1, -1)
        chain = graphs.get(cache, graphs.DraftChainGraph, llama, b, k - 1, float(temperature), bucket, latency)
        qs, toks = chain.run(t0, metas[1:], u[1:])
        return torch.cat([t0.view(b, 1), toks], dim=1), torch.cat([q0.view(b, 1, -1), qs], dim=1)

    def rollback(self, seq_id: int, keep: int) -> None:
        self.cache.truncate(seq_id, min(self.cache.length(seq_id), keep))

    def release(self, seq_id: int) -> None:
        self.cache.free(seq_id)


class UniformDraft:
    """Drafts ids uniformly at random with q = 1/V everywhere.  Almost every
    draft is rejected, so this exercises the residual-sampling path; the loop's
    output distribution must still be the target's."""

    def __init__(self, vocab_size: int) -> None:
        self.vocab_size = vocab_size

    def prefill(self, seq_ids: list[int], prompts: list[list[int]]) -> None:
        pass

    def propose(self, seq_ids: list[int], contexts: list[list[int]], k: int, temperature: float,
                generator: torch.Generator) -> tuple[torch.Tensor, torch.Tensor]:
        dev = torch.device("cuda", torch.cuda.current_device())
        q = torch.full((len(seq_ids), k, self.vocab_size), 1.0 / self.vocab_size, device=dev)
        gdev = generator.device if generator is not None else torch.device("cpu")
        draft = torch.randint(0, self.vocab_size, (len(seq_ids), k), generator=generator, device=gdev)
        return draft, q

    def rollback(self, seq_id: int, keep: int) -> None:
        pass

    def release(self, seq_id: int) -> None:
        pass


def run(model, cache: KVCache, seq_ids: list[int], chunks: list[list[int]] | torch.Tensor,
        latency_split: bool = False, temperature: float | None = None) -> torch.Tensor:
    """Forward right-padded chunks; returns the logits after each row's last
    real token, [B, V] (their probabilities at `temperature`, when given).
    `chunks` may also be a [B, w] id tensor already on the device (every row
    w tokens long)."""
    if isinstance(chunks, torch.Tensor):
        return forward(model, cache, seq_ids, chunks, [chunks.shape[1]] * chunks.shape[0], last_only=True,
                       latency_split=latency_split, temperature=temperature)
    n_new = [len(c) for c in chunks]
    width = max(n_new)
    input_ids = torch.tensor([c + [0] * (width - len(c)) for c in chunks], dtype=torch.int64)
    return forward(model, cache, seq_ids, input_ids, n_new, last_only=True, latency_split=latency_split,
                   temperature=temperature)
