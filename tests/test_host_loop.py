"""The round driver's host logic (spec/loop.py) on the CPU: its device calls
(prefill run, probabilities, sample, verify, accept_reject) are replaced by
the oracle's CPU functions, its caches and drafters by the oracle's, so what
is checked is the driver's own bookkeeping -- token cut, statistics, cache
rollback points, release order, events -- against outputs and statistics
the reference itself produced (tests/golden/loop_tiny.json) and against the
oracle's restatement of the reference loop."""
import pytest
import torch

import oracle.accept as oa
import oracle.draft as od
import oracle.kv as okv
import oracle.loop as ol
import oracle.sampling as osamp
import spec.loop as loop
from helpers import golden
from tiny_models import early_exit, oracle_model, random_prompts, reference_tiny, weights_sha

FIELDS = ("rounds", "accepted", "drafted", "attempts", "accepts", "emitted_per_round", "drafted_per_round")


@pytest.fixture(scope="module")
def tiny():
    return reference_tiny(0, torch.float64)


@pytest.fixture
def on_cpu(monkeypatch):
    """spec.loop with its device calls served by the oracle."""
    monkeypatch.setattr(loop, "run", od.run)
    monkeypatch.setattr(loop, "probabilities", osamp.probabilities)
    monkeypatch.setattr(loop, "sample", od.sample)
    monkeypatch.setattr(loop, "verify", od.verify)
    monkeypatch.setattr(loop, "accept_reject", oa.accept_reject)
    return loop


def cache_for(model, bs=4, nb=4096):
    return okv.KVCache.for_model(oracle_model(model).config, nb, bs, torch.float64)


class LoggingCache:
    """An oracle cache that records the calls the driver makes."""

    def __init__(self, inner, log):
        self.inner, self.log = inner, log

    def __getattr__(self, name):
        return getattr(self.inner, name)

    def add(self, s):
        self.log.append(("add", s))
        self.inner.add(s)

    def free(self, s):
        self.log.append(("free", s))
        self.inner.free(s)

    def truncate(self, s, n):
        self.log.append(("truncate", s, n))
        self.inner.truncate(s, n)


def test_driver_reproduces_reference_outputs_and_stats(on_cpu, tiny):
    data = golden("loop_tiny.json")
    assert weights_sha(tiny) == data["weights_sha256"]
    target = oracle_model(tiny)
    draft = oracle_model(early_exit(tiny))
    for run in data["runs"]:
        drafter = (od.ModelDraft(draft, cache_for(early_exit(tiny))) if run["drafter"] == "model"
                   else od.NGramDraft(256))
        out, stats = on_cpu.generate(target, cache_for(tiny), drafter, data["prompts"], data["max_new"], data["k"],
                                     temperature=run["temperature"],
                                     generator=torch.Generator().manual_seed(run["seed"]))
        assert out == run["outputs"]
        for f in FIELDS:
            assert getattr(stats, f) == run[f], f
        assert stats.discarded == stats.drafted - stats.accepted


@pytest.mark.parametrize("temperature,k", [(0.0, 4), (0.0, 1), (1.0, 3), (0.8, 8)])
def test_driver_matches_oracle_loop_with_eos_and_cache_calls(on_cpu, tiny, temperature, k):
    """eos inside a round's window, a budget that cuts a round short, and
    the exact sequence of cache calls (adds, rollbacks to context - 1,
    releases in row order) against the oracle's restatement of the loop."""
    target = oracle_model(tiny)
    draft = oracle_model(early_exit(tiny))
    prompts = random_prompts(7, 256, seed=31)
    # an eos id some row reaches mid-run: a token the same run emits without
    # an eos (the draws agree up to the first eos, so that row stops there)
    free_run, _ = ol.generate(target, cache_for(tiny), od.ModelDraft(draft, cache_for(early_exit(tiny))), prompts, 17,
                              k, temperature=temperature, generator=torch.Generator().manual_seed(9))
    eos = free_run[2][5]
    logs = {"ours": [], "oracle": []}
    outs = {}
    for who, gen_fn in (("ours", on_cpu.generate), ("oracle", ol.generate)):
        cache = LoggingCache(cache_for(tiny), logs[who])
        drafter = od.ModelDraft(draft, cache_for(early_exit(tiny)))
        outs[who] = gen_fn(target, cache, drafter, prompts, 17, k, temperature=temperature,
                           generator=torch.Generator().manual_seed(9), eos_id=eos)
    (o1, s1), (o2, s2) = outs["ours"], outs["oracle"]
    assert o1 == o2
    assert any(o and o[-1] == eos and len(o) < 17 for o in o1)
    for f in FIELDS:
        assert getattr(s1, f) == getattr(s2, f), f
    # the oracle releases a finished row before truncating the next; both
    # orders are the reference's (per row, in row order)
    assert logs["ours"] == logs["oracle"]


def test_events_fire_in_order_once(on_cpu, tiny):
    target = oracle_model(tiny)
    draft = oracle_model(early_exit(tiny))
    seen = []
    on_cpu.generate(target, cache_for(tiny), od.ModelDraft(draft, cache_for(early_exit(tiny))),
                    random_prompts(3, 256, seed=5), 12, 4, on_event=seen.append)
    assert seen == ["first_token", "draft_prefilled", "first_round"]


def test_one_token_budget_releases_before_any_round(on_cpu, tiny):
    target = oracle_model(tiny)
    log = []
    cache = LoggingCache(cache_for(tiny), log)
    out, stats = on_cpu.generate(target, cache, od.NGramDraft(256), random_prompts(3, 256, seed=6), 1, 4)
    assert [len(o) for o in out] == [1, 1, 1]
    assert stats.rounds == 0 and stats.emitted_per_round == []
    assert log == [("add", 0), ("add", 1), ("add", 2), ("free", 0), ("free", 1), ("free", 2)]


def test_stats_tally_matches_the_reference_bookkeeping():
    """SpecStats.tally against the reference's record/trim rules
    (spec/loop.py:107-120), for every n and cut at k = 4."""
    k = 4
    for n in range(k + 1):
        for emitted in range(n + 2):
            st = loop.SpecStats(k)
            st.tally(n, emitted)
            assert st.drafted == k and st.accepted == n
            assert st.attempts == [1 if i <= n else 0 for i in range(k)]
            assert st.accepts == [1 if i < n else 0 for i in range(k)]
            assert st.emitted_per_round == [emitted] and st.drafted_per_round == [min(n, emitted)]
            assert all(type(x) is int for x in st.attempts + st.accepts)


@pytest.mark.parametrize("tokens,room,eos,want", [
    ([5, 6, 7], 10, None, [5, 6, 7]), ([5, 6, 7], 2, None, [5, 6]), ([5, 6, 7], 10, 6, [5, 6]),
    ([5, 6, 7], 1, 6, [5]), ([6, 6], 5, 6, [6]), ([5], 0, None, [])])
def test_cut(tokens, room, eos, want):
    assert loop._cut(tokens, room, eos) == want


@pytest.fixture
def plain_on_cpu(monkeypatch):
    """baselines.cached_autoregressive with its forward served by the oracle."""
    import oracle.forward as of
    from baselines import cached_autoregressive as ca

    monkeypatch.setattr(ca, "forward", of.forward)
    monkeypatch.setattr(ca, "next_token", osamp.next_token)
    return ca


def test_plain_decoder_single_and_batched_match_oracle_greedy(plain_on_cpu, tiny):
    target = oracle_model(tiny)
    prompts = random_prompts(6, 256, seed=12)
    want = [ol.greedy(target, cache_for(tiny), p, 14) for p in prompts]
    assert [plain_on_cpu.generate(target, cache_for(tiny), p, 14) for p in prompts] == want
    assert plain_on_cpu.generate_batch(target, cache_for(tiny), prompts, 14) == want
    # eos: each row stops at its first eos, batched or alone, and its cache
    # sequence is gone afterwards
    eos = want[3][4]
    cut = [w[: w.index(eos) + 1] if eos in w else w for w in want]
    cache = cache_for(tiny)
    assert plain_on_cpu.generate_batch(target, cache, prompts, 14, eos_id=eos) == cut
    assert cache.tables == {}
    assert [plain_on_cpu.generate(target, cache_for(tiny), p, 14, eos_id=eos) for p in prompts] == cut
    assert plain_on_cpu.generate(target, cache_for(tiny), prompts[0], 0) == []


def test_plain_decoder_sampled_draw_order(plain_on_cpu, tiny):
    """At T > 0 a batch draws once per live row per step, in row order: a
    batch of one draws exactly as single-row decoding does."""
    target = oracle_model(tiny)
    p = random_prompts(1, 256, seed=13)[0]
    one = plain_on_cpu.generate(target, cache_for(tiny), p, 9, temperature=0.7,
                                generator=torch.Generator().manual_seed(3))
    batch = plain_on_cpu.generate_batch(target, cache_for(tiny), [p], 9, temperature=0.7,
                                        generator=torch.Generator().manual_seed(3))
    assert batch == [one] and len(one) == 9
