"""Prompt-lookup drafting on the GPU (reference: spec/ngram.py).

The match itself is the specdec_ngram_lookup kernel: one workgroup per row
finds, for n = min(max_n, len-1) down to 1, the most recent earlier
occurrence of the context's last n tokens and copies the k tokens that
followed it (the copy reads its own output once it runs past the end).
Without a match the last token is repeated k times.

NGramDraft keeps every sequence's history in a device buffer and uploads only
the tokens appended since its previous call, so a round costs one small
host-to-device copy, one lookup launch and one one-hot launch.
"""
from __future__ import annotations

import torch

from specdec import ops


class _History:
    """int32 [rows, cap] token histories on the GPU, one row per sequence."""

    def __init__(self, device: torch.device, rows: int = 16, cap: int = 4096) -> None:
        self.device = device
        self.buf = torch.zeros(rows, cap, dtype=torch.int32, device=device)
        self.row_of: dict[int, int] = {}
        self.length: dict[int, int] = {}
        # the tokens a row holds, and the context list they came from
        self.tokens: dict[int, list[int]] = {}
        self.source: dict[int, list[int]] = {}
        self._free = list(range(rows - 1, -1, -1))

    def _grow(self, rows: int, cap: int) -> None:
        old = self.buf
        new = torch.zeros(max(rows, old.shape[0]), max(cap, old.shape[1]), dtype=torch.int32, device=self.device)
        new[: old.shape[0], : old.shape[1]].copy_(old)
        self._free = list(range(new.shape[0] - 1, old.shape[0] - 1, -1)) + self._free
        self.buf = new

    def row(self, seq_id: int) -> int:
        r = self.row_of.get(seq_id)
        if r is None:
            if not self._free:
                self._grow(2 * self.buf.shape[0], self.buf.shape[1])
            r = self.row_of[seq_id] = self._free.pop()
            self.length[seq_id] = 0
        return r

    def release(self, seq_id: int) -> None:
        r = self.row_of.pop(seq_id, None)
        if r is not None:
            self._free.append(r)
            self.length.pop(seq_id, None)
            self.tokens.pop(seq_id, None)
            self.source.pop(seq_id, None)

    def sync(self, seq_ids: list[int], contexts: list[list[int]]) -> torch.Tensor:
        """Bring each sequence's device row up to its context; returns the
        int32 lengths [B] on the device.  Only the tokens past the row's are
        uploaded when the context extends them.  The same list object as last
        time (this package's round loop appends to its contexts in place) is
        taken to have been appended to, which is checked at the row's last
        token only: O(new tokens) host work per row, whatever the context's
        length.  A different list (the reference's loop builds a new one each
        round) is compared with the row's tokens on the host, O(length); a
        list that does not extend them is uploaded whole.  A caller that
        edits a context it passed before anywhere but at its end must pass a
        new list, or release the sequence first."""
        need = max(len(c) for c in contexts)
        if need > self.buf.shape[1]:
            self._grow(self.buf.shape[0], max(need, 2 * self.buf.shape[1]))
        flat_idx: list[int] = []
        values: list[int] = []
        cap = self.buf.shape[1]
        for seq_id, ctx in zip(seq_ids, contexts):
            r = self.row(seq_id)
            have = self.length[seq_id]
            held = self.tokens.setdefault(seq_id, [])
            if have > len(ctx):  # shorter: keep the rows' tokens if it is their prefix
                have = len(ctx) if ctx == held[:len(ctx)] else 0
            elif have > 0 and (ctx is not self.source.get(seq_id) or ctx[have - 1] != held[have - 1]):
                if ctx[:have] != held[:have]:
                    have = 0
            del held[have:]
            held.extend(ctx[have:])
            if have < len(ctx):
                base = r * cap
                flat_idx.extend(range(base + have, base + len(ctx)))
                values.extend(ctx[have:])
            self.length[seq_id] = len(ctx)
            self.source[seq_id] = ctx
        if values:
            host = torch.tensor([flat_idx, values], dtype=torch.int64).pin_memory()
            dev = host.to(self.device, non_blocking=True)
            self.buf.view(-1)[dev[0]] = dev[1].to(torch.int32)
        return torch.tensor([len(c) for c in contexts], dtype=torch.int32).pin_memory().to(self.device,
                                                                                             non_blocking=True)


def _check_contexts(contexts: list[list[int]]) -> None:
    for ctx in contexts:
        if len(ctx) == 0:
            raise IndexError("list index out of range: lookup needs a non-empty context")


class NGramDraft:
    """Prompt-lookup drafting (Saxena 2023) with a deterministic proposal, so q
    is the one-hot of the proposed token.  Accept-reject stays exact: the
    guarantee holds for any q the token was drawn from, a point mass included."""

    def __init__(self, vocab_size: int, max_n: int = 3, device=None) -> None:
        self.vocab_size = vocab_size
        self.max_n = max_n
        self._device = torch.device(device) if device is not None else None
        self._hist: _History | None = None
        self.last_match: torch.Tensor | None = None  # int32 [B, 2] of the latest propose

    def _history(self) -> _History:
        if self._hist is None:
            dev = self._device or torch.device("cuda", torch.cuda.current_device())
            self._hist = _History(dev)
        return self._hist

    def prefill(self, seq_ids: list[int], prompts: list[list[int]]) -> None:
        _check_contexts(prompts)
        self._history().sync(seq_ids, prompts)

    def propose(self, seq_ids: list[int], contexts: list[list[int]], k: int, temperature: float,
                generator: torch.Generator) -> tuple[torch.Tensor, torch.Tensor]:
        _check_contexts(contexts)
        hist = self._history()
        lengths = hist.sync(seq_ids, contexts)
        rows = [hist.row_of[s] for s in seq_ids]
        view = hist.buf if rows == list(range(rows[0], rows[0] + len(rows))) else None
        if view is not None:
            view = hist.buf[rows[0]: rows[0] + len(rows)]
        else:
            view = hist.buf[torch.tensor(rows, device=hist.device)]
        draft, match = ops.ngram_lookup(view, lengths, k, self.max_n)
        self.last_match = match
        return draft, ops.one_hot(draft, self.vocab_size)

    def rollback(self, seq_id: int, keep: int) -> None:
        pass

    def release(self, seq_id: int) -> None:
        if self._hist is not None:
            self._hist.release(seq_id)


def lookup_batch(contexts: list[list[int]], k: int, max_n: int, device=None) -> tuple[list[list[int]], list[tuple[int, int]]]:
    """Proposals and (match start, n) for independent contexts, one launch."""
    _check_contexts(contexts)
    dev = torch.device(device) if device is not None else torch.device("cuda", torch.cuda.current_device())
    cap = max(len(c) for c in contexts)
    hist = torch.zeros(len(contexts), cap, dtype=torch.int32)
    for i, c in enumerate(contexts):
        hist[i, : len(c)] = torch.tensor(c, dtype=torch.int32)
    lengths = torch.tensor([len(c) for c in contexts], dtype=torch.int32)
    draft, match = ops.ngram_lookup(hist.to(dev), lengths.to(dev), k, max_n)
    return draft.cpu().tolist(), [tuple(m) for m in match.cpu().tolist()]


def lookup(context: list[int], k: int, max_n: int) -> list[int]:
    """spec/ngram.py:32-45 for one context (one kernel launch)."""
    return lookup_batch([context], k, max_n)[0][0]
