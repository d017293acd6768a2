"""N-gram lookup kernel vs the oracle, the reference's literals and golden rows."""
import hashlib
import json

import pytest
import torch

import oracle.ngram as on
from helpers import golden
from workloads import planted_rows
from spec.ngram import NGramDraft, lookup, lookup_batch

pytestmark = pytest.mark.gpu


def test_reference_literals():
    assert lookup([1, 2, 3, 4, 1, 2], k=2, max_n=3) == [3, 4]
    assert lookup([1, 2, 3, 1, 2], k=5, max_n=2) == [3, 1, 2, 3, 1]
    ctx = [7, 8, 9, 1, 8, 5, 7, 8]
    assert lookup(ctx, k=1, max_n=2) == [9]
    assert lookup(ctx, k=1, max_n=1) == [5]
    assert lookup([1, 4, 2, 4, 3, 4], k=1, max_n=1) == [3]
    assert lookup([1, 2, 3], k=3, max_n=3) == [3, 3, 3]


def test_golden_rows():
    for case in golden("ngram.json")["cases"]:
        rows = case["rows"]
        if rows is None:
            rows = planted_rows(*case["gen"])
            assert hashlib.sha256(json.dumps(rows).encode()).hexdigest() == case["rows_sha"]
        got, _ = lookup_batch(rows, case["k"], case["max_n"])
        assert got == case["out"], (case["gen"], case["k"], case["max_n"])


@pytest.mark.parametrize("length", [2048, 4096, 8192])
def test_config3_batch16_matches_oracle_with_positions(length):
    rows = planted_rows(16, length, 49152, seed=length)
    got, match = lookup_batch(rows, 4, 3)
    for row, g, m in zip(rows, got, match):
        want, start, n = on.lookup_match(row, 4, 3)
        assert g == want
        assert tuple(m) == (start, n)


@pytest.mark.parametrize("vocab", [2, 3, 7])
def test_small_vocab_random_rows_all_n(vocab):
    g = torch.Generator().manual_seed(vocab)
    rows = [torch.randint(0, vocab, (int(n),), generator=g).tolist()
            for n in torch.randint(1, 40, (64,), generator=g)]
    for k in (0, 1, 4, 9):
        for max_n in (0, 1, 2, 3, 5, 8):
            got, match = lookup_batch(rows, k, max_n)
            for row, gt, m in zip(rows, got, match):
                want, start, n = on.lookup_match(row, k, max_n)
                assert gt == want and tuple(m) == (start, n), (row, k, max_n)


def test_drafter_incremental_history_matches_full_lookup():
    """NGramDraft uploads only appended tokens; proposals equal lookup on the
    whole context every round, and q is the one-hot of the proposal."""
    rows = planted_rows(4, 600, 50, seed=3)
    drafter = NGramDraft(64)
    ctxs = [r[:200] for r in rows]
    for step in range(0, 300, 37):
        ctxs = [r[: 200 + step] for r in rows]
        draft, q = drafter.propose([0, 1, 2, 3], ctxs, 4, 0.0, None)
        want = [on.lookup(c, 4, 3) for c in ctxs]
        assert draft.cpu().tolist() == want
        assert torch.equal(q.cpu(), torch.nn.functional.one_hot(torch.tensor(want), 64).float())
    drafter.release(1)
    draft, _ = drafter.propose([1], [rows[1][:50]], 4, 0.0, None)
    assert draft.cpu().tolist() == [on.lookup(rows[1][:50], 4, 3)]


def test_reused_sequence_id_with_another_context_is_uploaded_again():
    """A sequence id reused for a different context of the same length and
    last token (the reference's NGramDraft keeps no state, so its proposal
    depends on the context alone): the history is re-uploaded, not reused."""
    a = [5, 6, 7, 1, 2, 3, 9, 1, 2, 3]
    b = [8, 8, 8, 1, 2, 4, 6, 1, 2, 3]  # same length and last tokens, other content
    drafter = NGramDraft(16)
    for ctx in (a, b, list(a), a[:7], b + [6]):
        draft, _ = drafter.propose([0], [ctx], 4, 0.0, None)
        assert draft.cpu().tolist() == [on.lookup(ctx, 4, 3)], ctx


@pytest.mark.parametrize("max_n", [9, 17, 64, 65, 100, 1000])
def test_any_max_n_matches_oracle(max_n):
    """max_n past the staged tail (64 tokens) and tile overlap: periodic rows
    agree over long spans (agreements that run out of the staged tokens read
    memory), random small-vocab rows over short ones; one row crosses the
    8192-position tile boundary."""
    g = torch.Generator().manual_seed(max_n)
    rows = [[i % 5 for i in range(300)], [i % 7 for i in range(8300)], [(i * 3) % 11 for i in range(150)]]
    rows += [torch.randint(0, 3, (int(n),), generator=g).tolist() for n in torch.randint(2, 120, (8,), generator=g)]
    for k in (1, 4):
        got, match = lookup_batch(rows, k, max_n)
        for row, gt, m in zip(rows, got, match):
            want, start, n = on.lookup_match(row, k, max_n)
            assert gt == want and tuple(m) == (start, n), (len(row), k, max_n)


@pytest.mark.parametrize("max_n", [0, 1, 3])
def test_one_token_histories_and_no_ngram(max_n):
    """Histories too short for any n-gram (one token), and max_n 0: no tile
    is scanned and the proposal repeats the last token."""
    rows = [[7], [1, 2, 1], [5, 6, 7, 5], [9, 9]]
    for k in (1, 4):
        got, match = lookup_batch(rows, k, max_n)
        for row, gt, m in zip(rows, got, match):
            want, start, n = on.lookup_match(row, k, max_n)
            assert gt == want and tuple(m) == (start, n), (row, k, max_n)


def test_lengths_past_the_row_are_taken_as_the_row():
    """A length beyond the history buffer's row stride (a caller's mistake
    the host cannot see: lengths live on the GPU) reads nothing outside the
    row: the kernel takes the row's whole stride as the history."""
    from specdec import ops

    g = torch.Generator().manual_seed(4)
    hist = torch.randint(0, 5, (3, 40), generator=g, dtype=torch.int32)
    want = [on.lookup_match(row.tolist(), 4, 3) for row in hist]
    lengths = torch.tensor([40, 41, 1 << 30], dtype=torch.int32)
    draft, match = ops.ngram_lookup(hist.cuda(), lengths.cuda(), 4, 3)
    for (w, start, n), gt, m in zip(want, draft.cpu().tolist(), match.cpu().tolist()):
        assert gt == w and tuple(m) == (start, n)


def test_empty_context_raises():
    with pytest.raises(IndexError):
        lookup([], 3, 3)


def _unique_row(length, first=100):
    return list(range(first, first + length))


def test_long_histories_across_lds_tiles():
    """Histories longer than one 8192-position tile: the scan walks tiles from
    the end and may stop only once the longest n has matched.  Cases: the
    only 3-gram match in the earliest tile, a more recent 2-gram that must
    not win over it, 3-grams whose aligned position sits on either side of a
    tile boundary, and lengths at the edge of one tile."""
    rows = []
    r = _unique_row(20000)
    r[-3:] = [1, 2, 3]
    r[10:13] = [1, 2, 3]
    rows.append(r)
    r = list(rows[0])
    r[15000:15002] = [2, 3]
    rows.append(r)
    for shift in (0, 1, 2, 3):
        r = _unique_row(20000)
        r[-3:] = [1, 2, 3]
        lo0 = 20000 - 8193  # first position of the last tile scanned first
        e = lo0 - shift
        r[e - 2: e + 1] = [1, 2, 3]
        rows.append(r)
    for length in (8192, 8193, 8194, 8195, 8255, 8256, 8257, 16387):
        r = _unique_row(length)
        r[-1] = r[0]  # a single 1-gram match at the very start
        rows.append(r)
        r = _unique_row(length)  # no match at all: the fallback
        rows.append(r)
    for k in (1, 4):
        got, match = lookup_batch(rows, k, 3)
        for row, g, m in zip(rows, got, match):
            want, start, n = on.lookup_match(row, k, 3)
            assert g == want and tuple(m) == (start, n), (len(row), start, n, tuple(m))
