"""Pins the oracle's model path: the cached forward against transformers'
own uncached forward (fp64), and the whole round loop against the golden
outputs and statistics the reference produced on its tiny model."""
import pytest
import torch

import oracle.forward as of
import oracle.kv as okv
from helpers import golden
from oracle.draft import ModelDraft, NGramDraft
from oracle.loop import generate, greedy
from tiny_models import early_exit, oracle_model, reference_tiny, weights_sha

TOL = 1e-10


@pytest.fixture(scope="module")
def tiny():
    return reference_tiny(0, torch.float64)


def cache_for(model, bs=4, nb=4096):
    m = oracle_model(model)
    return okv.KVCache.for_model(m.config, nb, bs, torch.float64)


@torch.no_grad()
def test_cached_forward_matches_hf_recompute(tiny):
    om = oracle_model(tiny)
    tokens = torch.randint(0, 256, (24,), generator=torch.Generator().manual_seed(1)).tolist()
    for bs in (1, 3, 16):
        cache = cache_for(tiny, bs)
        cache.add(0)
        got = of.forward(om, cache, [0], torch.tensor([tokens[:5]]), [5])[0]
        want = tiny(torch.tensor([tokens[:5]]), use_cache=False).logits[0]
        assert (got - want).abs().max().item() <= TOL
        for t in range(5, 24):
            step = of.forward(om, cache, [0], torch.tensor([[tokens[t]]]), [1])[0, 0]
            full = tiny(torch.tensor([tokens[: t + 1]]), use_cache=False).logits[0, -1]
            assert (step - full).abs().max().item() <= TOL


@torch.no_grad()
def test_padded_mixed_batch_matches_hf(tiny):
    om = oracle_model(tiny)
    gen = torch.Generator().manual_seed(2)
    seqs = [torch.randint(0, 256, (n,), generator=gen).tolist() for n in (3, 9, 6)]
    cache = cache_for(tiny, 4)
    for s in range(3):
        cache.add(s)
    for r, n_new in enumerate([[3, 9, 6], [1, 3, 2], [2, 1, 1], [1, 1, 4]]):
        if r:
            for s, n in zip(seqs, n_new):
                s.extend(torch.randint(0, 256, (n,), generator=gen).tolist())
        chunks = [s[len(s) - n:] for s, n in zip(seqs, n_new)]
        w = max(n_new)
        out = of.forward(om, cache, [0, 1, 2], torch.tensor([c + [0] * (w - len(c)) for c in chunks]), n_new)
        for b, (s, n) in enumerate(zip(seqs, n_new)):
            want = tiny(torch.tensor([s]), use_cache=False).logits[0, len(s) - n:]
            assert (out[b, :n] - want).abs().max().item() <= TOL


def test_loop_reproduces_reference_outputs_and_stats(tiny):
    data = golden("loop_tiny.json")
    assert weights_sha(tiny) == data["weights_sha256"]
    target = oracle_model(tiny)
    draft = oracle_model(early_exit(tiny))
    for run in data["runs"]:
        drafter = (ModelDraft(draft, cache_for(early_exit(tiny))) if run["drafter"] == "model"
                   else NGramDraft(256))
        out, stats = generate(target, cache_for(tiny), drafter, data["prompts"], data["max_new"], data["k"],
                              temperature=run["temperature"], generator=torch.Generator().manual_seed(run["seed"]))
        assert out == run["outputs"]
        for f in ("rounds", "accepted", "drafted", "attempts", "accepts", "emitted_per_round", "drafted_per_round"):
            assert getattr(stats, f) == run[f], f


def test_greedy_spec_equals_plain_greedy(tiny):
    target = oracle_model(tiny)
    draft = oracle_model(early_exit(tiny))
    prompts = golden("loop_tiny.json")["prompts"]
    out, _ = generate(target, cache_for(tiny), ModelDraft(draft, cache_for(early_exit(tiny))), prompts, 20, 4)
    assert out == [greedy(target, cache_for(tiny), p, 20) for p in prompts]
