"""Seeded synthetic inputs of the benchmark workloads.

* `planted_rows`: token histories with copies of earlier spans planted into
  them (prompt lookup's config-3 histories and the batched decode prompts).
* `accept_inputs`: a target/draft probability pair with draft tokens sampled
  from the draft distribution (the accept-reject workload).

Pure Python/torch on the CPU; the same seeds give the same inputs on every
machine, which is what lets golden fixtures be regenerated from a seed.
"""
from __future__ import annotations

import random

import torch


def planted_rows(n_rows: int, length: int, vocab: int, seed: int, cover: float = 0.3) -> list[list[int]]:
    """Integer histories, iid uniform over [0, vocab), with about `cover` of
    the positions overwritten by copies of earlier spans (span lengths 8..64),
    so that prompt lookup finds matches of every length."""
    rng = random.Random(seed)
    rows = []
    for _ in range(n_rows):
        row = [rng.randrange(vocab) for _ in range(length)]
        covered = 0
        while covered < cover * length:
            span = rng.randint(8, 64)
            if length < 2 * span + 2:
                break
            src = rng.randrange(0, length - 2 * span)
            dst = rng.randrange(src + span, length - span + 1)
            row[dst:dst + span] = row[src:src + span]
            covered += span
        rows.append(row)
    return rows


def accept_inputs(dtype: torch.dtype, b: int, k: int, v: int, noise: float, seed: int):
    """Target probabilities p [b, k+1, v] and draft probabilities q [b, k, v]
    (softmax of N(0, 2^2) logits, the draft's first k rows perturbed by
    N(0, noise^2)), computed in fp64 and cast to `dtype`, and draft tokens
    [b, k] drawn from q."""
    g = torch.Generator().manual_seed(seed)
    tl = torch.randn(b, k + 1, v, generator=g, dtype=torch.float64) * 2.0
    dl = tl[:, :k] + torch.randn(b, k, v, generator=g, dtype=torch.float64) * noise
    p = torch.softmax(tl, -1).to(dtype)
    q = torch.softmax(dl, -1).to(dtype)
    draft = torch.multinomial(q.reshape(-1, v).double(), 1, generator=g).view(b, k)
    return p, q, draft
