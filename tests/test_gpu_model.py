"""The model path on the GPU: cached forward vs transformers' uncached
forward, greedy identity of the speculative loop, rollback, the bonus token,
and the loop at T > 0 against the oracle loop on the same weights."""
import math

import pytest
import torch

import oracle.kv as okv
from baselines import cached_autoregressive
from cache.kv import KVCache
from lm.forward import forward
from oracle.draft import ModelDraft as OModelDraft
from oracle.loop import generate as ogenerate
from spec.draft import ModelDraft, UniformDraft
from spec.loop import generate
from spec.ngram import NGramDraft
from tiny_models import early_exit, oracle_model, random_prompts, tiny64

pytestmark = pytest.mark.gpu
MAX_NEW = 24


@pytest.fixture(scope="module")
def tiny():
    return tiny64(0, torch.float32)


@pytest.fixture(scope="module")
def tiny_draft(tiny):
    return early_exit(tiny)


def new_cache(model, num_blocks=4096, block_size=4, dtype=torch.float32):
    return KVCache.for_model(model.config, num_blocks=num_blocks, block_size=block_size, dtype=dtype, device="cuda")


@torch.no_grad()
def recompute(model, tokens):
    return model(torch.tensor([tokens]), use_cache=False).logits[0]


@pytest.fixture(scope="module")
def prompts(tiny):
    return random_prompts(40, tiny.config.vocab_size, seed=10)


@pytest.fixture(scope="module")
def expected(tiny, prompts):
    return [cached_autoregressive.generate(tiny, new_cache(tiny), p, MAX_NEW) for p in prompts]


@pytest.mark.parametrize("block_size", [1, 3, 16])
def test_incremental_matches_recompute(tiny, block_size):
    tokens = torch.randint(0, 256, (40,), generator=torch.Generator().manual_seed(1)).tolist()
    cache = new_cache(tiny, 256, block_size)
    cache.add(0)
    got = forward(tiny, cache, [0], torch.tensor([tokens[:5]]), [5])[0].cpu()
    worst = (got - recompute(tiny, tokens[:5])).abs().max().item()
    for t in range(5, 40):
        step = forward(tiny, cache, [0], torch.tensor([[tokens[t]]]), [1])[0, 0].cpu()
        worst = max(worst, (step - recompute(tiny, tokens[: t + 1])[-1]).abs().max().item())
    assert worst < 2e-4, worst


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_norm_weights_folded_into_projections(dtype):
    """Non-unit RMSNorm weights (input, post-attention and final), which the
    forward folds into the projections' columns: prefill (a separate norm
    kernel) and decode steps (norms finished in the attention and SiLU*up
    kernels, bf16 only) against transformers' uncached forward of the same
    model.  Unit weights, as a fresh model has, would leave a fold that
    scales rows instead of columns unseen."""
    model = tiny64(3, torch.float32)
    g = torch.Generator().manual_seed(4)
    with torch.no_grad():
        for name, w in model.named_parameters():
            if name.endswith("norm.weight"):
                w.copy_(0.25 + 1.5 * torch.rand(w.shape, generator=g))
    model = model.to(dtype)
    tokens = torch.randint(0, 256, (24,), generator=torch.Generator().manual_seed(5)).tolist()
    cache = new_cache(model, 256, 16, dtype)
    cache.add(0)
    got = [forward(model, cache, [0], torch.tensor([tokens[:20]]), [20])[0, -1].float().cpu()]
    for t in range(20, 24):
        got.append(forward(model, cache, [0], torch.tensor([[tokens[t]]]), [1])[0, 0].float().cpu())
    want = [recompute(model, tokens[: t + 1])[-1].float() for t in range(19, 24)]
    for a, b in zip(got, want):
        if dtype == torch.float32:
            assert (a - b).abs().max().item() < 2e-4 * max(1.0, b.abs().max().item())
        else:  # bf16 roundings apart (a misplaced fold is off by tens of percent)
            assert ((a - b).norm() / b.norm()).item() < 0.05
    if dtype == torch.float32:  # the greedy choice agrees with transformers' at every step
        assert [a.argmax().item() for a in got] == [b.argmax().item() for b in want]


@pytest.mark.parametrize("block_size", [1, 4, 16])
def test_padded_batch_of_mixed_lengths(tiny, block_size):
    gen = torch.Generator().manual_seed(2)
    seqs = [torch.randint(0, 256, (n,), generator=gen).tolist() for n in (3, 9, 6)]
    cache = new_cache(tiny, 256, block_size)
    for s in range(3):
        cache.add(s)
    worst = 0.0
    for r, n_new in enumerate([[3, 9, 6], [1, 3, 2], [2, 1, 1], [1, 1, 4]]):
        if r:
            for s, n in zip(seqs, n_new):
                s.extend(torch.randint(0, 256, (n,), generator=gen).tolist())
        chunks = [s[len(s) - n:] for s, n in zip(seqs, n_new)]
        w = max(n_new)
        logits = forward(tiny, cache, [0, 1, 2], torch.tensor([c + [0] * (w - len(c)) for c in chunks]), n_new).cpu()
        for b, (s, n) in enumerate(zip(seqs, n_new)):
            worst = max(worst, (logits[b, :n] - recompute(tiny, s)[len(s) - n:]).abs().max().item())
    assert worst < 2e-4, worst


@pytest.mark.parametrize("block_size", [1, 4])
def test_truncate_then_append(tiny, block_size):
    gen = torch.Generator().manual_seed(3)
    prefix = torch.randint(0, 256, (10,), generator=gen).tolist()
    rejected = torch.randint(0, 256, (4,), generator=gen).tolist()
    replacement = torch.randint(0, 256, (3,), generator=gen).tolist()
    cache = new_cache(tiny, 256, block_size)
    cache.add(0)
    forward(tiny, cache, [0], torch.tensor([prefix]), [10])
    forward(tiny, cache, [0], torch.tensor([rejected]), [4])
    cache.truncate(0, 11)
    logits = forward(tiny, cache, [0], torch.tensor([replacement]), [3])[0].cpu()
    want = recompute(tiny, prefix + rejected[:1] + replacement)[-3:]
    assert cache.length(0) == 14
    assert (logits - want).abs().max().item() < 2e-4


def test_cached_greedy_equals_oracle_greedy(tiny, prompts, expected):
    """Plain greedy on the GPU == the oracle's CPU greedy (same fp32 weights)."""
    from oracle.loop import greedy

    om = oracle_model(tiny)
    for p, want in zip(prompts[:10], expected[:10]):
        assert greedy(om, okv.KVCache.for_model(om.config, 4096, 4, torch.float32), p, MAX_NEW) == want


def test_identical_one_at_a_time(tiny, tiny_draft, prompts, expected):
    accepted = drafted = 0
    for prompt, want in zip(prompts, expected):
        out, stats = generate(tiny, new_cache(tiny), ModelDraft(tiny_draft, new_cache(tiny_draft)), [prompt],
                              MAX_NEW, k=4)
        assert out[0] == want
        accepted += stats.accepted
        drafted += stats.drafted
    assert 0.1 < accepted / drafted < 0.95, accepted / drafted


@pytest.mark.parametrize("batch", [8, 13])
def test_identical_batched(tiny, tiny_draft, prompts, expected, batch):
    for i in range(0, len(prompts), batch):
        out, _ = generate(tiny, new_cache(tiny), ModelDraft(tiny_draft, new_cache(tiny_draft)),
                          prompts[i:i + batch], MAX_NEW, k=4)
        assert out == expected[i:i + batch]


@pytest.mark.parametrize("batch,k", [(1, 4), (2, 4), (3, 4), (1, 15)])
def test_bf16_identical_while_every_projection_is_row_invariant(batch, k):
    """bf16, calls of at most 16 rows (the verify's B * (k+1) and plain
    decoding's B): every projection runs on specdec_linear, whose rows do not
    depend on the other rows of the call, so speculative greedy decoding
    emits plain greedy decoding's tokens at these batches too.  (Larger
    verify calls run on hipBLASLt, whose bits depend on the call's row
    count; there, as on the reference's GPU path, only fp32 is exact.)"""
    model = tiny64(5, torch.bfloat16)
    draft = early_exit(model)
    ps = random_prompts(6, model.config.vocab_size, seed=11, low=20, high=40)
    for i in range(0, len(ps), batch):
        chunk = ps[i:i + batch]
        want = cached_autoregressive.generate_batch(model, new_cache(model, 512, 16, torch.bfloat16), chunk, MAX_NEW)
        out, _ = generate(model, new_cache(model, 512, 16, torch.bfloat16),
                          ModelDraft(draft, new_cache(draft, 512, 16, torch.bfloat16)), chunk, MAX_NEW, k=k)
        assert out == want, (batch, k, i)


@pytest.mark.parametrize("k", [1, 2, 3, 8])
def test_identical_across_draft_lengths(tiny, tiny_draft, prompts, expected, k):
    out, _ = generate(tiny, new_cache(tiny), ModelDraft(tiny_draft, new_cache(tiny_draft)), prompts[:16], MAX_NEW, k=k)
    assert out == expected[:16]


def test_copy_of_target_accepts_everything(tiny, prompts, expected):
    out, stats = generate(tiny, new_cache(tiny), ModelDraft(tiny, new_cache(tiny)), prompts[:16], MAX_NEW, k=4)
    assert out == expected[:16]
    assert stats.accepted == stats.drafted


def test_uniform_draft_is_still_exact(tiny, prompts, expected):
    out, stats = generate(tiny, new_cache(tiny), UniformDraft(256), prompts[:16], MAX_NEW, k=4,
                          generator=torch.Generator().manual_seed(0))
    assert out == expected[:16]
    assert stats.accepted / stats.drafted < 0.05


def test_ngram_draft_is_still_exact(tiny, prompts, expected):
    out, _ = generate(tiny, new_cache(tiny), NGramDraft(256), prompts[:16], MAX_NEW, k=4)
    assert out == expected[:16]


def test_eos_stops_mid_window(tiny, tiny_draft, prompts, expected):
    want = expected[0]
    eos = want[5]
    cut = want[: want.index(eos) + 1]
    out, _ = generate(tiny, new_cache(tiny), ModelDraft(tiny_draft, new_cache(tiny_draft)), [prompts[0]], MAX_NEW, k=4,
                      eos_id=eos)
    assert out[0] == cut


class ScriptedDraft:
    """Proposes the target's greedy continuation for the first j positions and
    a wrong token after, so every round accepts exactly j drafts."""

    def __init__(self, reference, prompt_len, j, vocab):
        self.reference, self.prompt_len, self.j, self.vocab = reference, prompt_len, j, vocab

    def prefill(self, seq_ids, prompts):
        pass

    def propose(self, seq_ids, contexts, k, temperature, generator):
        done = len(contexts[0]) - self.prompt_len
        right = self.reference[done:done + k] + [0] * k
        draft = [right[i] if i < self.j else (right[i] + 1) % self.vocab for i in range(k)]
        tokens = torch.tensor([draft])
        return tokens, torch.nn.functional.one_hot(tokens, self.vocab).float()

    def rollback(self, seq_id, keep):
        pass

    def release(self, seq_id):
        pass


@pytest.mark.parametrize("j", range(5))
def test_exactly_j_accepted_every_round(tiny, j):
    prompt = random_prompts(1, 256, seed=3)[0]
    want = cached_autoregressive.generate(tiny, new_cache(tiny), prompt, 30 + 5)
    out, stats = generate(tiny, new_cache(tiny), ScriptedDraft(want, len(prompt), j, 256), [prompt], 30, k=4)
    assert out[0] == want[:30]
    assert stats.accepts[:j] == stats.attempts[:j]
    assert all(a == 0 for a in stats.accepts[j:])
    assert all(e == j + 1 for e in stats.emitted_per_round[:-1])


def test_drafted_per_round_counts(tiny):
    _, stats = generate(tiny, new_cache(tiny), ModelDraft(tiny, new_cache(tiny)), [[1, 2, 3, 4]], 13, k=4)
    assert stats.emitted_per_round == [5, 5, 2]
    assert stats.drafted_per_round == [4, 4, 2]


@pytest.mark.parametrize(("k", "max_new"), [(1, 20), (4, 21), (4, 23), (7, 30)])
def test_full_acceptance_emits_k_plus_one(tiny, k, max_new):
    prompt = random_prompts(1, 256, seed=5)[0]
    want = cached_autoregressive.generate(tiny, new_cache(tiny), prompt, max_new)
    out, stats = generate(tiny, new_cache(tiny), ModelDraft(tiny, new_cache(tiny)), [prompt], max_new, k=k)
    assert out[0] == want
    assert stats.rounds == math.ceil((max_new - 1) / (k + 1))


def test_bonus_with_copy_draft_never_rejects_at_t1(tiny):
    prompts = random_prompts(10, 256, seed=6)
    _, stats = generate(tiny, new_cache(tiny), ModelDraft(tiny, new_cache(tiny)), prompts, 20, k=4, temperature=1.0,
                        generator=torch.Generator().manual_seed(0))
    assert stats.accepted == stats.drafted


@pytest.mark.parametrize("temperature", [1.0, 0.8])
def test_sampled_loop_matches_oracle_loop(tiny, tiny_draft, temperature):
    """Same weights, same generator seed: the GPU loop emits the oracle loop's
    tokens and statistics (fp32 on both sides)."""
    prompts = random_prompts(6, 256, seed=4)
    target, draft = oracle_model(tiny), oracle_model(tiny_draft)
    want_out, want = ogenerate(target, okv.KVCache.for_model(target.config, 4096, 4, torch.float32),
                               OModelDraft(draft, okv.KVCache.for_model(draft.config, 4096, 4, torch.float32)),
                               prompts, 20, 4, temperature=temperature, generator=torch.Generator().manual_seed(7))
    got_out, got = generate(tiny, new_cache(tiny), ModelDraft(tiny_draft, new_cache(tiny_draft)), prompts, 20, 4,
                            temperature=temperature, generator=torch.Generator().manual_seed(7))
    assert got_out == want_out
    assert (got.rounds, got.accepted, got.attempts, got.accepts) == (want.rounds, want.accepted, want.attempts,
                                                                     want.accepts)


@pytest.mark.parametrize("temperature", [0.0, 1.0])
def test_graph_replay_equals_eager_launches(tiny, tiny_draft, monkeypatch, temperature):
    """The captured verify and draft graphs produce the same tokens and
    statistics as the same kernels launched one by one."""
    prompts = random_prompts(5, 256, seed=12)
    runs = []
    for flag in ("0", "1"):
        monkeypatch.setenv("SPECDEC_GRAPHS", flag)
        out, stats = generate(tiny, new_cache(tiny), ModelDraft(tiny_draft, new_cache(tiny_draft)), prompts, 30, 4,
                              temperature=temperature, generator=torch.Generator().manual_seed(3))
        runs.append((out, stats.rounds, stats.accepted, stats.emitted_per_round))
    assert runs[0] == runs[1]


def test_graphs_are_reused_across_requests(tiny, tiny_draft, prompts, expected):
    """One cache pair serving several requests in turn: graphs captured for the
    first are replayed for the next, and outputs stay exact."""
    tc, dc = new_cache(tiny), new_cache(tiny_draft)
    for p, want in zip(prompts[:6], expected[:6]):
        out, _ = generate(tiny, tc, ModelDraft(tiny_draft, dc), [p], MAX_NEW, k=4)
        assert out[0] == want
    assert len(tc.graphs) >= 1 and len(dc.graphs) >= 1
    assert tc.allocator.num_used == 0 and dc.allocator.num_used == 0


class CheckedDraft:
    """A ModelDraft whose every proposal is checked against a recompute of
    the draft model without a cache on the context it was drafted from: a
    cache that kept rejected tokens (or lost accepted ones) would propose
    from the wrong context."""

    def __init__(self, model, cache):
        self.model, self.inner = model, ModelDraft(model, cache)

    def prefill(self, seq_ids, prompts):
        self.inner.prefill(seq_ids, prompts)

    def propose(self, seq_ids, contexts, k, temperature, generator):
        draft, q = self.inner.propose(seq_ids, contexts, k, temperature, generator)
        draft_h, q_h = draft.cpu(), q.cpu()
        for row, ctx in enumerate(contexts):
            logits = recompute(self.model, ctx + draft_h[row, :-1].tolist())[-k:]
            assert torch.equal(q_h[row], torch.nn.functional.one_hot(logits.argmax(-1), q_h.shape[-1]).float())
        return draft, q

    def rollback(self, seq_id, keep):
        self.inner.rollback(seq_id, keep)

    def release(self, seq_id):
        self.inner.release(seq_id)


def test_draft_cache_conditions_on_the_right_tokens(tiny, tiny_draft):
    prompts = random_prompts(6, tiny.config.vocab_size, seed=4)
    _, stats = generate(tiny, new_cache(tiny), CheckedDraft(tiny_draft, new_cache(tiny_draft)), prompts, MAX_NEW, k=4)
    # partial and full acceptance both occur, so both rollback cases were checked
    assert 0 < stats.accepted < stats.drafted
    assert any(e == 5 for e in stats.emitted_per_round)


class RecordingDraft(ModelDraft):
    """Remembers the token it proposed for each absolute position."""

    def __init__(self, model, cache):
        super().__init__(model, cache)
        self.proposed = {}

    def propose(self, seq_ids, contexts, k, temperature, generator):
        draft, q = super().propose(seq_ids, contexts, k, temperature, generator)
        for i, tok in enumerate(draft[0].tolist()):
            self.proposed[len(contexts[0]) + i] = tok
        return draft, q


def lenient_verify(delta):
    """A verification that is known to be wrong: a drafted token whose logit
    is within delta of the row's maximum counts as the target's choice."""
    from lm.forward import forward as fwd

    def verify(target, cache, seq_ids, contexts, draft, temperature):
        draft = draft.cpu()
        ids = torch.cat([torch.tensor([[c[-1]] for c in contexts]), draft], dim=1)
        logits = fwd(target, cache, seq_ids, ids, [ids.shape[1]] * len(seq_ids)).float()
        choice = logits.argmax(-1)
        d = draft.to(logits.device)
        at_draft = logits[:, :-1].gather(-1, d[..., None]).squeeze(-1)
        near = at_draft >= logits[:, :-1].max(-1).values - delta
        choice[:, :-1] = torch.where(near, d, choice[:, :-1])
        return torch.nn.functional.one_hot(choice, logits.shape[-1]).float()

    return verify


def test_lenient_verification_shows_as_draft_biased_divergences(tiny, tiny_draft, prompts, expected, monkeypatch):
    """The loop calls spec.loop.verify at run time, so a patched verify that
    accepts near-tied drafts takes effect: outputs then part from plain greedy
    decoding, and every first divergence lands on the draft's token -- what
    the greedy identity tests would catch."""
    monkeypatch.setattr("spec.loop.verify", lenient_verify(0.5))
    covered = hits = 0
    for prompt, want in zip(prompts, expected):
        drafter = RecordingDraft(tiny_draft, new_cache(tiny_draft))
        out, _ = generate(tiny, new_cache(tiny), drafter, [prompt], MAX_NEW, k=4)
        at = next((i for i, (x, y) in enumerate(zip(out[0], want)) if x != y), None)
        if at is None:
            continue
        pos = len(prompt) + at
        if pos in drafter.proposed:
            covered += 1
            hits += out[0][at] == drafter.proposed[pos]
    assert covered >= 3
    assert hits == covered


@pytest.mark.parametrize("batch", [1, 3, 8])
def test_batched_plain_decoding_matches_one_at_a_time(tiny, batch):
    prompts = random_prompts(24, 256, seed=11, low=1, high=40)
    want = [cached_autoregressive.generate(tiny, new_cache(tiny), p, 12) for p in prompts]
    cache = new_cache(tiny)
    for i in range(0, len(prompts), batch):
        assert cached_autoregressive.generate_batch(tiny, cache, prompts[i:i + batch], 12) == want[i:i + batch]
    assert cache.allocator.num_used == 0 and not cache.tables


def test_batched_plain_decoding_drops_a_row_at_eos(tiny):
    prompts = [[5, 6, 7], list(range(30, 60))]
    full = [cached_autoregressive.generate(tiny, new_cache(tiny), p, 12) for p in prompts]
    eos = full[0][3]
    want = [cached_autoregressive.generate(tiny, new_cache(tiny), p, 12, eos_id=eos) for p in prompts]
    assert len(want[0]) <= 4
    assert cached_autoregressive.generate_batch(tiny, new_cache(tiny), prompts, 12, eos_id=eos) == want
