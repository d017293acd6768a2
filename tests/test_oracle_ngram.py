"""Pins oracle.ngram: the reference's literals, golden rows written by the
reference, and an independent brute-force definition."""
import hashlib
import json

import torch

import oracle.ngram as on
from helpers import golden
from workloads import planted_rows


def brute(ctx, k, max_n):
    """Largest n, then largest start, by enumerating every (n, start) pair."""
    best = None
    for n in range(1, min(max_n, len(ctx) - 1) + 1):
        for s in range(0, len(ctx) - n):
            if ctx[s:s + n] == ctx[len(ctx) - n:]:
                if best is None or (n, s) > best:
                    best = (n, s)
    if best is None:
        return [ctx[-1]] * k, -1, 0
    n, s = best
    src = ctx[s + n:]
    return [src[i % len(src)] for i in range(k)], s, n


def test_reference_literals():
    assert on.lookup([1, 2, 3, 4, 1, 2], 2, 3) == [3, 4]
    assert on.lookup([1, 2, 3, 1, 2], 5, 2) == [3, 1, 2, 3, 1]
    assert on.lookup([7, 8, 9, 1, 8, 5, 7, 8], 1, 2) == [9]
    assert on.lookup([7, 8, 9, 1, 8, 5, 7, 8], 1, 1) == [5]
    assert on.lookup([1, 4, 2, 4, 3, 4], 1, 1) == [3]
    assert on.lookup([1, 2, 3], 3, 3) == [3, 3, 3]


def test_golden_rows():
    for case in golden("ngram.json")["cases"]:
        rows = case["rows"]
        if rows is None:
            rows = planted_rows(*case["gen"])
            assert hashlib.sha256(json.dumps(rows).encode()).hexdigest() == case["rows_sha"]
        assert [on.lookup(r, case["k"], case["max_n"]) for r in rows] == case["out"]


def test_matches_brute_force_on_small_vocab():
    g = torch.Generator().manual_seed(0)
    for _ in range(400):
        n = int(torch.randint(1, 30, (1,), generator=g))
        ctx = torch.randint(0, 3, (n,), generator=g).tolist()
        for k in (1, 4, 7):
            for max_n in (1, 2, 3, 4):
                assert on.lookup_match(ctx, k, max_n) == brute(ctx, k, max_n)
