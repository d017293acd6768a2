"""Oracle of spec/draft.py and spec/verify.py (test infrastructure)."""
import torch

from oracle.accept import sample_inverse_cdf
from oracle.forward import forward
from oracle.sampling import probabilities


def sample(probs, generator):
    """spec/draft.py:27-29"""
    u = torch.rand(probs.shape[0], generator=generator, dtype=probs.dtype)
    return sample_inverse_cdf(probs, u)


def run(model, cache, seq_ids, chunks):
    """spec/draft.py:87-92"""
    n_new = [len(c) for c in chunks]
    width = max(n_new)
    input_ids = torch.tensor([c + [0] * (width - len(c)) for c in chunks])
    return forward(model, cache, seq_ids, input_ids, n_new, last_only=True)


class ModelDraft:
    """spec/draft.py:32-62"""

    def __init__(self, model, cache):
        self.model, self.cache = model, cache

    def prefill(self, seq_ids, prompts):
        for s in seq_ids:
            self.cache.add(s)
        run(self.model, self.cache, seq_ids, prompts)

    def propose(self, seq_ids, contexts, k, temperature, generator):
        pending = [ctx[self.cache.length(s):] for s, ctx in zip(seq_ids, contexts)]
        tokens, qs = [], []
        for _ in range(k):
            q = probabilities(run(self.model, self.cache, seq_ids, pending), temperature)
            token = sample(q, generator)
            tokens.append(token)
            qs.append(q)
            pending = [[t] for t in token.tolist()]
        return torch.stack(tokens, dim=1), torch.stack(qs, dim=1)

    def rollback(self, seq_id, keep):
        self.cache.truncate(seq_id, min(self.cache.length(seq_id), keep))

    def release(self, seq_id):
        self.cache.free(seq_id)


class NGramDraft:
    """spec/ngram.py:4-29"""

    def __init__(self, vocab_size, max_n=3):
        self.vocab_size, self.max_n = vocab_size, max_n

    def prefill(self, seq_ids, prompts):
        pass

    def propose(self, seq_ids, contexts, k, temperature, generator):
        from oracle.ngram import lookup

        draft = torch.tensor([lookup(ctx, k, self.max_n) for ctx in contexts])
        return draft, torch.nn.functional.one_hot(draft, self.vocab_size).float()

    def rollback(self, seq_id, keep):
        pass

    def release(self, seq_id):
        pass


def verify(target, cache, seq_ids, contexts, draft, temperature):
    """spec/verify.py:9-30"""
    for seq_id, ctx in zip(seq_ids, contexts):
        if cache.length(seq_id) != len(ctx) - 1:
            raise RuntimeError(f"seq {seq_id}: target cache holds {cache.length(seq_id)}, expected {len(ctx) - 1}")
    last = torch.tensor([[ctx[-1]] for ctx in contexts])
    input_ids = torch.cat([last, draft], dim=1)
    logits = forward(target, cache, seq_ids, input_ids, [input_ids.shape[1]] * len(seq_ids))
    return probabilities(logits, temperature)
