"""A seeded sweep of n-gram lookup calls against the oracle: ragged batches of
1-16 histories whose lengths cluster at the kernel's tile edges (8192 and
8256 positions, their multiples) as well as anywhere up to 20000, vocabularies
from 2 tokens (a match at nearly every position) to 49152 (almost none) with
planted copies, k 1-8 and max_n 0-6.  Proposals and (match start, n)
bit-exact."""
import random

import pytest

import oracle.ngram as on
from spec.ngram import lookup_batch

pytestmark = pytest.mark.gpu

EDGES = [1, 2, 3, 8191, 8192, 8193, 8255, 8256, 8257, 16384, 16385, 16448, 16449]


def _row(rng, length, vocab):
    row = [rng.randrange(vocab) for _ in range(length)]
    # planted copies of earlier spans, as config 3 has
    for _ in range(rng.randint(0, 4)):
        if length < 20:
            break
        n = rng.randint(2, min(64, length // 2))
        src = rng.randrange(0, length - n)
        dst = rng.randrange(0, length - n + 1)
        row[dst:dst + n] = row[src:src + n]
    return row


def _cases(n=30, seed=8):
    rng = random.Random(seed)
    out = []
    for i in range(n):
        vocab = rng.choice([2, 5, 50, 49152])
        rows = rng.randint(1, 16)
        lengths = [rng.choice(EDGES) if rng.random() < 0.5 else rng.randint(1, 20000) for _ in range(rows)]
        k, max_n = rng.choice([1, 4, 8]), rng.randint(0, 6)
        out.append(pytest.param(vocab, lengths, k, max_n, 300 + i, id=f"{i}-v{vocab}-r{rows}-k{k}-n{max_n}"))
    return out


@pytest.mark.parametrize("vocab,lengths,k,max_n,seed", _cases())
def test_random_batches_match_oracle(vocab, lengths, k, max_n, seed):
    rng = random.Random(seed)
    rows = [_row(rng, n, vocab) for n in lengths]
    got, match = lookup_batch(rows, k, max_n)
    for row, gt, m in zip(rows, got, match):
        want, start, n = on.lookup_match(row, k, max_n)
        assert gt == want and tuple(m) == (start, n), (len(row), k, max_n)
