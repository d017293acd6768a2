"""Batched sampled speculative decoding (8 and 32 rows, T = 0.8, k = 4 and 8,
the 135M-shaped model drafter and the n-gram drafter, 1024-token prompts
with ~30% planted repetition) against the oracle's restatement of the
reference loop on the same fp32 weights: SmolLM2-1.7B layer shapes for the
target and SmolLM2-135M shapes for the draft, two layers each so the CPU
oracle finishes in seconds, vocab 49152.  The graphs' context buckets are
shrunk to 1040 keys so that the 32 new tokens cross a bucket (a recapture
at 2080 keys, five 512-key splits) as well as 16-token block boundaries.

Every sampled decision of both runs is recorded: the first token (inverse
CDF of the prefill's softmax), each draft token (inverse CDF of the draft
softmax, model drafter) and each round's accept-reject (u_accept, u_residual
drawn from the same generator in the same order).  The runs must agree
token for token and in every SpecStats field.  At V = 49152 a decision can
legitimately part two correct fp32 implementations: the GPU's and the CPU's
forwards round differently (about 1e-6 relative), and an inverse-CDF target
that lies closer than that to a CDF boundary picks the neighbouring token.
So if the runs part, the first differing decision must be explained:
  * on the GPU's own inputs, the oracle makes the GPU's decision (kernel
    parity, with the 1e-6 accept band);
  * the GPU's probabilities equal the oracle's within 1e-4 relative;
  * the decision's margin on the oracle's inputs (|u q(x) - p(x)| / p(x) for
    the accept test, the distance of the inverse-CDF target to the boundary
    between the two tokens over the total mass) is below 1e-4;
and everything emitted before it must agree."""
import pytest
import torch

import oracle.accept as oa
import oracle.draft as od
import oracle.forward as of
import oracle.kv as okv
import oracle.loop as ol
import spec.loop as loop
from cache.kv import KVCache
from lm import graphs
from lm.model import SMOLLM2_135M, SMOLLM2_1_7B, Llama, random_state_dict
from spec.draft import ModelDraft
from spec.ngram import NGramDraft
from workloads import planted_rows

pytestmark = pytest.mark.gpu
V = 49152
PROMPT, NEW, T = 1024, 32, 0.8
BUCKET = PROMPT + 16  # context bucket of the captured graphs in these tests
REL = 1e-4  # fp32 forward tolerance (GPU vs CPU probabilities, decision margins)


def shapes():
    return SMOLLM2_1_7B.replace(num_hidden_layers=2), SMOLLM2_135M.replace(num_hidden_layers=2)


def oracle_model(shape, state):
    cfg = of.Config(shape.vocab_size, shape.hidden_size, shape.num_hidden_layers, shape.num_attention_heads,
                    shape.num_key_value_heads, shape.intermediate_size, shape.head_dim, shape.rms_norm_eps,
                    shape.rope_theta, shape.tie_word_embeddings)
    return of.Model(cfg, {k: v.cpu() for k, v in state.items()})


@pytest.fixture(scope="module")
def models():
    ts, ds = shapes()
    t_state = random_state_dict(ts, 0, "cuda", torch.float32)
    d_state = random_state_dict(ds, 1, "cuda", torch.float32)
    return ((Llama.from_state_dict(ts, t_state), Llama.from_state_dict(ds, d_state)),
            (oracle_model(ts, t_state), oracle_model(ds, d_state)))


def record_run(generate_fn, module, target, cache, drafter, prompts, k, seed):
    """Run generate_fn with module.sample / module.accept_reject wrapped to
    record every sampled decision; returns (outputs, stats, records)."""
    records = {"first": None, "rounds": []}
    real_sample, real_accept = module.sample, module.accept_reject
    gen = torch.Generator().manual_seed(seed)
    state = {}

    def sample(probs, generator):
        saved = generator.get_state()
        tokens = real_sample(probs, generator)
        u = torch.rand(probs.shape[0], generator=torch.Generator().set_state(saved), dtype=probs.dtype)
        records["first"] = (probs.float().cpu(), u, tokens.cpu())
        return tokens

    def accept_reject(p, q, draft, generator=None):
        b, kk = draft.shape
        ua = torch.rand(b, kk, generator=generator, dtype=p.dtype)
        ur = torch.rand(b, generator=generator, dtype=p.dtype)
        v = real_accept(p, q, draft, u_accept=ua, u_residual=ur)
        records["rounds"].append({"p": p.float().cpu(), "q": q.float().cpu(), "draft": draft.cpu(), "ua": ua,
                                  "ur": ur, "n": v.n_accepted.cpu(), "x": v.next_token.cpu(),
                                  "draft_state": state["before_propose"]})
        state["before_propose"] = generator.get_state()
        return v

    def on_event(name):
        if name == "draft_prefilled":
            state["before_propose"] = gen.get_state()

    module.sample, module.accept_reject = sample, accept_reject
    try:
        kw = {"on_event": on_event} if generate_fn is loop.generate else {}
        if generate_fn is not loop.generate:
            # the oracle loop has no events: its draft proposals start right
            # after the first token's draw, as the reference's do
            def first_then_mark(probs, generator):
                out = sample(probs, generator)
                state["before_propose"] = generator.get_state()
                return out
            module.sample = first_then_mark
        out, stats = generate_fn(target, cache, drafter, prompts, NEW, k, temperature=T, generator=gen, **kw)
    finally:
        module.sample, module.accept_reject = real_sample, real_accept
    return out, stats, records


def cdf_margin(probs: torch.Tensor, u: float, x1: int, x2: int) -> float:
    """Distance, over the total mass, from the inverse-CDF target u * total to
    the nearest CDF boundary between tokens x1 and x2 (fp64 cumsum)."""
    cdf = probs.double().cumsum(-1)
    lo, hi = min(x1, x2), max(x1, x2)
    target = u * cdf[-1].item()
    return (cdf[lo:hi] - target).abs().min().item() / cdf[-1].item()


def close(a: torch.Tensor, b: torch.Tensor) -> bool:
    return bool(((a - b).abs() <= REL * b.abs() + 1e-9).all())


def explain_round(g, c, k):
    """First round whose accept decision differs, same drafts: explained?"""
    assert close(g["p"], c["p"]) and close(g["q"], c["q"]), "GPU and CPU probabilities differ beyond fp32 rounding"
    # kernel parity: the oracle on the GPU's inputs makes the GPU's decision
    v = oa.accept_reject(g["p"], g["q"], g["draft"], u_accept=g["ua"], u_residual=g["ur"])
    band = oa.accept_reject_exclusion(g["p"], g["q"], g["draft"], g["ua"], g["ur"])
    same = (v.n_accepted == g["n"]) & (v.next_token == g["x"])
    assert bool((same | band).all()), "the accept kernel disagrees with the oracle on identical inputs"
    margins = []
    for row in torch.nonzero((g["n"] != c["n"]) | (g["x"] != c["x"])).flatten().tolist():
        n = min(int(g["n"][row]), int(c["n"][row]))
        x = int(c["draft"][row, n]) if n < k else None
        if int(g["n"][row]) != int(c["n"][row]):  # the accept test at position n flipped
            px, qx = c["p"][row, n, x].double().item(), c["q"][row, n, x].double().item()
            margins.append(abs(float(c["ua"][row, n]) * qx - px) / px)
            continue
        # same n, different residual sample: the boundary between the tokens
        pr, qr = c["p"][row, n], (c["q"][row, n] if n < k else torch.zeros_like(c["p"][row, n]))
        r = oa.residual_distribution(pr[None], qr[None])[0]
        margins.append(cdf_margin(r, float(c["ur"][row]), int(g["x"][row]), int(c["x"][row])))
    return margins


@pytest.mark.timeout(900)
@pytest.mark.parametrize("B,drafter,k", [(8, "model", 4), (8, "model", 8), (8, "ngram", 4), (8, "ngram", 8),
                                         (32, "model", 8), (32, "ngram", 8)])
def test_batched_sampled_loop_matches_oracle(models, monkeypatch, B, drafter, k):
    (target, draft), (otarget, odraft) = models
    print(f"[case] batched sampled B={B} T={T} k={k} {drafter}", flush=True)
    monkeypatch.setattr(graphs, "BUCKET", BUCKET)
    buckets = set()
    real_bucket_for = graphs.bucket_for
    monkeypatch.setattr(graphs, "bucket_for", lambda m: buckets.add(real_bucket_for(m)) or real_bucket_for(m))
    prompts = planted_rows(B, PROMPT, V, seed=B * 100 + k)
    ts, ds = shapes()
    blocks = B * ((PROMPT + NEW + 2 * k + 32) // 16 + 2)
    gpu_drafter = (ModelDraft(draft, KVCache.for_model(ds, blocks, 16, torch.float32, "cuda")) if drafter == "model"
                   else NGramDraft(V))
    ocfg_t, ocfg_d = otarget.config, odraft.config
    cpu_drafter = (od.ModelDraft(odraft, okv.KVCache.for_model(ocfg_d, blocks, 16, torch.float32))
                   if drafter == "model" else od.NGramDraft(V))
    g_out, g_stats, g_rec = record_run(loop.generate, loop, target,
                                       KVCache.for_model(ts, blocks, 16, torch.float32, "cuda"), gpu_drafter,
                                       prompts, k, seed=5)
    c_out, c_stats, c_rec = record_run(ol.generate, ol, otarget, okv.KVCache.for_model(ocfg_t, blocks, 16,
                                                                                       torch.float32),
                                       cpu_drafter, prompts, k, seed=5)
    assert g_stats.rounds > 0
    assert len(buckets) >= 2, buckets  # the run crossed a context bucket

    # first token
    gp, gu, gx = g_rec["first"]
    cp, cu, cx = c_rec["first"]
    assert torch.equal(gu, cu) and close(gp, cp)
    if not torch.equal(gx, cx):
        rows = torch.nonzero(gx != cx).flatten().tolist()
        worst = max(cdf_margin(cp[r], float(cu[r]), int(gx[r]), int(cx[r])) for r in rows)
        assert worst < REL, worst
        print(f"[parted] at the first token, margin {worst:.2e}")
        return
    # rounds, until the first decision that differs
    for i, (g, c) in enumerate(zip(g_rec["rounds"], c_rec["rounds"])):
        assert torch.equal(g["draft_state"], c["draft_state"])
        if not torch.equal(g["draft"], c["draft"]):
            # a draft token differs (model drafter): the draft's own inverse-CDF draw
            assert drafter == "model"
            gen = torch.Generator().set_state(c["draft_state"])
            u = torch.stack([torch.rand(g["draft"].shape[0], generator=gen) for _ in range(k)], dim=1)
            first = torch.nonzero((g["draft"] != c["draft"]).any(dim=0)).flatten()[0].item()
            rows = torch.nonzero(g["draft"][:, first] != c["draft"][:, first]).flatten().tolist()
            assert torch.equal(g["draft"][:, :first], c["draft"][:, :first])
            assert close(g["q"][:, first], c["q"][:, first])
            gx = od.sample_inverse_cdf(g["q"][:, first], u[:, first].float())
            assert torch.equal(gx, g["draft"][:, first]), "the draft sampler disagrees with the oracle"
            worst = max(cdf_margin(c["q"][r, first], float(u[r, first]), int(g["draft"][r, first]),
                                   int(c["draft"][r, first])) for r in rows)
            assert worst < REL, worst
            print(f"[parted] round {i}: draft token, margin {worst:.2e}")
            break
        assert torch.equal(g["ua"], c["ua"]) and torch.equal(g["ur"], c["ur"])
        if not (torch.equal(g["n"], c["n"]) and torch.equal(g["x"], c["x"])):
            margins = explain_round(g, c, k)
            assert max(margins) < REL, margins
            print(f"[parted] round {i}: accept decision, margins {margins}")
            break
        assert close(g["p"], c["p"]) and close(g["q"], c["q"])
    else:
        assert g_out == c_out
        for f in ("rounds", "accepted", "drafted", "attempts", "accepts", "emitted_per_round", "drafted_per_round"):
            assert getattr(g_stats, f) == getattr(c_stats, f), f
        print(f"[identical] {g_stats.rounds} rounds, acceptance {g_stats.accepted / g_stats.drafted:.3f}")
        return
    # parted at round i: every per-(row, round) statistic before it agrees
    settled = sum(int(((r["n"] >= 0)).sum()) for r in g_rec["rounds"][:i])
    assert g_stats.emitted_per_round[:settled] == c_stats.emitted_per_round[:settled]
    assert g_stats.drafted_per_round[:settled] == c_stats.drafted_per_round[:settled]
