"""End-to-end greedy identity at SmolLM2 shapes (layer count reduced so the
CPU oracle finishes in seconds): target with 1.7B layer shapes (hidden 2048,
32/32 heads x 64, MLP 8192, RoPE theta 130000, vocab 49152, tied), draft
with 135M layer shapes (hidden 576, 9/3 heads, MLP 1536), random N(0, 0.02)
weights, 2 layers each.

fp32: the GPU speculative loop, GPU plain greedy decoding and the oracle's
fp32 greedy decoding (the reference's fp32 path, restated on the CPU) emit
the same tokens.  bf16: speculative output equals plain greedy output on
the GPU, token for token."""
import pytest
import torch

import oracle.forward as of
import oracle.kv as okv
from baselines import cached_autoregressive
from cache.kv import KVCache
from lm.model import SMOLLM2_135M, SMOLLM2_1_7B, Llama, random_state_dict
from oracle.loop import greedy
from spec.draft import ModelDraft
from spec.loop import generate

pytestmark = pytest.mark.gpu
V = 49152


def shapes():
    return SMOLLM2_1_7B.replace(num_hidden_layers=2), SMOLLM2_135M.replace(num_hidden_layers=2)


def oracle_model(shape, state):
    cfg = of.Config(shape.vocab_size, shape.hidden_size, shape.num_hidden_layers, shape.num_attention_heads,
                    shape.num_key_value_heads, shape.intermediate_size, shape.head_dim, shape.rms_norm_eps,
                    shape.rope_theta, shape.tie_word_embeddings)
    return of.Model(cfg, {k: v.cpu() for k, v in state.items()})


def prompts(n=3, length=64):
    g = torch.Generator().manual_seed(21)
    return [torch.randint(0, V, (length,), generator=g).tolist() for _ in range(n)]


def caches(t_shape, d_shape, dtype):
    return (KVCache.for_model(t_shape, 64, 16, dtype, "cuda"), KVCache.for_model(d_shape, 64, 16, dtype, "cuda"))


@pytest.mark.parametrize("k", [4])
def test_fp32_spec_equals_plain_equals_oracle(k):
    ts, ds = shapes()
    t_state = random_state_dict(ts, 0, "cpu", torch.float32)
    d_state = random_state_dict(ds, 1, "cpu", torch.float32)
    target = Llama.from_state_dict(ts, t_state, device="cuda")
    draft = Llama.from_state_dict(ds, d_state, device="cuda")
    om = oracle_model(ts, t_state)
    for p in prompts():
        tc, dc = caches(ts, ds, torch.float32)
        out, _ = generate(target, tc, ModelDraft(draft, dc), [p], 24, k=k)
        plain = cached_autoregressive.generate(target, KVCache.for_model(ts, 64, 16, torch.float32, "cuda"), p, 24)
        ref = greedy(om, okv.KVCache.for_model(om.config, 64, 16, torch.float32), p, 24)
        assert out[0] == plain == ref


def test_bf16_spec_equals_plain():
    ts, ds = shapes()
    target = Llama.random(ts, 0, "cuda", torch.bfloat16)
    draft = Llama.random(ds, 1, "cuda", torch.bfloat16)
    for p in prompts(4, 96):
        tc, dc = caches(ts, ds, torch.bfloat16)
        out, _ = generate(target, tc, ModelDraft(draft, dc), [p], 40, k=4)
        plain = cached_autoregressive.generate(target, KVCache.for_model(ts, 64, 16, torch.bfloat16, "cuda"), p, 40)
        assert out[0] == plain


def test_bf16_spec_equals_plain_with_norm_weights():
    """The same identity with non-unit RMSNorm weights in both models: the
    weights folded into the projections (rounded once into bf16 weights)
    serve the verify and plain decoding alike, so the outputs still agree."""
    ts, ds = shapes()

    def perturbed(shape, seed):
        state = random_state_dict(shape, seed, "cuda", torch.bfloat16)
        g = torch.Generator(device="cuda").manual_seed(seed + 100)
        for name, w in state.items():
            if name.endswith("norm.weight"):
                w.copy_((0.5 + torch.rand(w.shape, generator=g, device="cuda")).to(w.dtype))
        return Llama.from_state_dict(shape, state)

    target, draft = perturbed(ts, 0), perturbed(ds, 1)
    for p in prompts(2, 96):
        tc, dc = caches(ts, ds, torch.bfloat16)
        out, _ = generate(target, tc, ModelDraft(draft, dc), [p], 40, k=4)
        plain = cached_autoregressive.generate(target, KVCache.for_model(ts, 64, 16, torch.bfloat16, "cuda"), p, 40)
        assert out[0] == plain


def test_bf16_exact_copy_draft_accepts_every_token():
    """The target as its own draft, computing as the verify does: every
    round accepts all k drafts and emits the bonus token (k + 1 tokens), and
    the output is plain greedy decoding's (reference tests/test_greedy_identity.py:58-61)."""
    ts, _ = shapes()
    target = Llama.random(ts, 0, "cuda", torch.bfloat16)
    p = prompts(1, 96)[0]
    tc, dc = caches(ts, ts, torch.bfloat16)
    out, stats = generate(target, tc, ModelDraft(target, dc, exact=True), [p], 41, k=4)
    plain = cached_autoregressive.generate(target, KVCache.for_model(ts, 64, 16, torch.bfloat16, "cuda"), p, 41)
    assert out[0] == plain
    assert stats.accepted == stats.drafted == 4 * stats.rounds
    assert stats.emitted_per_round == [5] * 8 and stats.rounds == 8
