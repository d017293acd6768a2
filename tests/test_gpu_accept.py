"""Accept-reject kernels vs the oracle and the reference's known answers."""
import dataclasses
from fractions import Fraction

import pytest
import torch

import oracle.accept as oa
import oracle.sampling as osamp
from helpers import golden
from lm.sampling import probabilities
from spec.accept import Verdict, accept_reject, host_draft, residual_distribution, sample_inverse_cdf

pytestmark = pytest.mark.gpu
V = 49152

P = [Fraction(4, 10), Fraction(3, 10), Fraction(2, 10), Fraction(1, 10), Fraction(0)]
Q = [Fraction(1, 10), Fraction(2, 10), Fraction(3, 10), Fraction(1, 10), Fraction(3, 10)]
ACCEPT = [Fraction(1), Fraction(1), Fraction(2, 3), Fraction(1), Fraction(0)]


def t64(xs):
    return torch.tensor([float(x) for x in xs], dtype=torch.float64)


def config1_logits(seed: int):
    """Target logits [5, V] ~ N(0, 2^2); draft = first 4 rows + N(0, 0.5^2)."""
    g = torch.Generator().manual_seed(seed)
    target = torch.randn(5, V, generator=g) * 2.0
    draft = target[:4] + torch.randn(4, V, generator=g) * 0.5
    return target, draft


@pytest.mark.parametrize("temperature", [0.0, 1.0, 0.8, 0.25])
def test_probabilities_match_torch_softmax(temperature):
    target, draft = config1_logits(0)
    x = torch.cat([target, draft])
    want = osamp.probabilities(x, temperature)
    got = probabilities(x.cuda(), temperature).cpu()
    if temperature == 0.0:
        assert torch.equal(got, want)
    else:
        assert torch.allclose(got, want, rtol=1e-5, atol=1e-12)
        assert (got.double().sum(-1) - 1).abs().max() < 1e-5


@pytest.mark.parametrize("vocab", [V, 1000, 1001, 49151, 70000])
def test_probabilities_into_strided_rows_with_argmax(vocab):
    """Writing into a row-strided view (the draft chain's q[:, i]) gives the
    same rows; at temperature 0 index_out holds each row's argmax, which is
    what an inverse-CDF draw from the one-hot row returns.  Vocabularies that
    are a multiple of 4 move as 16-byte vectors, 1001 and 49151 element by
    element; 70000 exceeds the register-resident row size and takes the
    streaming loop."""
    from specdec import ops

    g = torch.Generator().manual_seed(vocab)
    x = (torch.randn(3, vocab, generator=g) * 3).cuda()
    for temperature in (0.0, 0.7, 1.0):
        want = osamp.probabilities(x.cpu(), temperature)
        q = torch.full((3, 2, vocab), -1.0, device="cuda")
        idx = torch.full((3, 2), -1, dtype=torch.int64, device="cuda")
        ops.probabilities(x, temperature, out=q[:, 1], index_out=idx[:, 1] if temperature == 0.0 else None)
        got = q[:, 1].cpu()
        assert torch.equal(q[:, 0].cpu(), torch.full((3, vocab), -1.0))
        if temperature == 0.0:
            assert torch.equal(got, want)
            assert idx[:, 1].cpu().tolist() == x.cpu().argmax(-1).tolist()
            assert idx[:, 0].cpu().tolist() == [-1, -1, -1]
            u = torch.rand(3, generator=g)
            assert sample_inverse_cdf(q[:, 1].contiguous(), u.cuda()).cpu().tolist() == idx[:, 1].cpu().tolist()
        else:
            assert torch.allclose(got, want, rtol=1e-5, atol=1e-12)


def test_probabilities_argmax_ties_go_to_lowest_id():
    x = torch.tensor([[1.0, 3.0, 3.0, 2.0], [5.0, 5.0, 5.0, 5.0], [-1.0, -2.0, -1.0, -3.0]])
    got = probabilities(x.cuda(), 0.0).cpu()
    assert got.argmax(-1).tolist() == [1, 0, 0]
    assert torch.equal(got.sum(-1), torch.ones(3))


def test_residual_matches_hand_computation():
    r = residual_distribution(t64(P), t64(Q)).cpu()
    assert torch.allclose(r, t64([Fraction(3, 4), Fraction(1, 4), 0, 0, 0]), atol=1e-15, rtol=0)


def test_scripted_uniforms():
    p = t64(P).expand(1, 2, 5)
    q = t64(Q).expand(1, 1, 5)
    draft = torch.tensor([[2]])

    def run(ua, ur):
        return accept_reject(p, q, draft, u_accept=torch.tensor([[ua]], dtype=torch.float64),
                             u_residual=torch.tensor([ur], dtype=torch.float64))

    accepted = run(0.6, 0.5)
    assert accepted.n_accepted.item() == 1 and accepted.next_token.item() == 1
    # the draft comes back with the verdict, as host int64 [B, k]
    assert host_draft(accepted).device.type == "cpu" and torch.equal(host_draft(accepted), draft)
    # the verdict itself is the reference's two-field frozen dataclass
    assert [f.name for f in dataclasses.fields(Verdict)] == ["n_accepted", "next_token"]
    assert len(dataclasses.astuple(accepted)) == 2
    rejected = run(0.7, 0.8)
    assert rejected.n_accepted.item() == 0 and rejected.next_token.item() == 1
    assert run(0.7, 0.5).next_token.item() == 0


def test_zero_target_mass_never_emitted():
    p = t64(P).expand(1000, 2, 5)
    q = t64(Q).expand(1000, 1, 5)
    verdict = accept_reject(p, q, torch.full((1000, 1), 4), generator=torch.Generator().manual_seed(0))
    assert verdict.n_accepted.sum().item() == 0
    assert set(verdict.next_token.tolist()) <= {0, 1}


def test_coupled_stream_reproduces_target_exactly():
    """The reference's exact-fractions test (tests/test_accept_toy.py:54-76) on the kernel."""
    n = 120
    grid = (torch.arange(n, dtype=torch.float64) + 0.5) / n
    u_accept = grid.repeat_interleave(n).unsqueeze(-1)
    u_residual = grid.repeat(n)
    p = t64(P).expand(n * n, 2, 5)
    q = t64(Q).expand(n * n, 1, 5)
    emitted = [Fraction(0)] * 5
    for y in range(5):
        draft = torch.full((n * n, 1), y)
        verdict = accept_reject(p, q, draft, u_accept=u_accept, u_residual=u_residual)
        first = torch.where(verdict.n_accepted == 1, draft[:, 0], verdict.next_token)
        assert Fraction(int(verdict.n_accepted.sum()), n * n) == ACCEPT[y]
        for x, count in enumerate(torch.bincount(first, minlength=5).tolist()):
            emitted[x] += Q[y] * Fraction(count, n * n)
    assert emitted == P


def test_greedy_reduces_to_argmax_verification():
    v = 5
    p = torch.nn.functional.one_hot(torch.tensor([[3, 1, 4]]), v).double()
    draft = torch.tensor([[3, 2]])
    q = torch.nn.functional.one_hot(draft, v).double()
    verdict = accept_reject(p, q, draft, generator=torch.Generator().manual_seed(0))
    assert verdict.n_accepted.item() == 1 and verdict.next_token.item() == 1
    all_match = accept_reject(p, torch.nn.functional.one_hot(torch.tensor([[3, 1]]), v).double(),
                              torch.tensor([[3, 1]]), generator=torch.Generator().manual_seed(0))
    assert all_match.n_accepted.item() == 2 and all_match.next_token.item() == 4


def test_inverse_cdf_skips_zero_mass():
    probs = torch.tensor([[0.0, 0.5, 0.0, 0.5, 0.0]], dtype=torch.float64)
    for u, expected in [(0.0, 1), (0.49, 1), (0.5, 3), (0.999, 3)]:
        assert sample_inverse_cdf(probs, torch.tensor([u], dtype=torch.float64)).item() == expected


def test_zero_draft_probability_raises():
    p = t64(P).expand(1, 2, 5)
    q = t64([0.5, 0.5, 0, 0, 0]).expand(1, 1, 5)
    with pytest.raises(ValueError):
        accept_reject(p, q, torch.tensor([[3]]), generator=torch.Generator().manual_seed(0))


@pytest.mark.parametrize("custom", [False, True])
@pytest.mark.parametrize("bad_id", [5, 6, -1])
def test_draft_id_outside_vocab_raises(custom, bad_id):
    """A draft id outside [0, V) is range-checked on the device (it is never
    used as an index) and raises ValueError on the fused path and on the
    custom-residual path alike; the reference's gather raises too."""
    p = t64(P).expand(1, 3, 5).contiguous()
    q = t64(Q).expand(1, 2, 5).contiguous()
    draft = torch.tensor([[2, bad_id]])
    kw = {"residual": lambda pp, qq: torch.clamp(pp - qq, min=0.0)} if custom else {}
    with pytest.raises(ValueError, match="vocabulary"):
        accept_reject(p, q, draft, generator=torch.Generator().manual_seed(0), **kw)
    torch.cuda.synchronize()


def _golden_inputs(case):
    from workloads import accept_inputs

    dtype = getattr(torch, case["dtype"])
    if case["p"] is not None:
        p = torch.tensor(case["p"], dtype=dtype)
        q = torch.tensor(case["q"], dtype=dtype)
        draft = torch.tensor(case["draft"])
    else:
        p, q, draft = accept_inputs(dtype, case["b"], case["k"], case["v"], case["noise"], case["input_seed"])
        assert draft.tolist() == case["draft"]
    return p, q, draft


@pytest.mark.parametrize("i", range(4))
def test_golden_generator_stream(i):
    """accept_reject with generator=: the reference's own outputs."""
    case = golden("accept_gen.json")["cases"][i]
    p, q, draft = _golden_inputs(case)
    verdict = accept_reject(p, q, draft, generator=torch.Generator().manual_seed(case["seed"]))
    assert verdict.n_accepted.tolist() == case["n_accepted"]
    assert verdict.next_token.tolist() == case["next_token"]


@pytest.mark.parametrize("seed", range(6))
@pytest.mark.parametrize("temperature", [1.0, 0.8])
def test_config1_matches_oracle(seed, temperature):
    """Config 1 shape (B=1, k=4, V=49152, fp32) plus a B=8 batch: n and token
    bit-exact except rows decided within 1e-6 of a threshold."""
    for b in (1, 8):
        g = torch.Generator().manual_seed(1000 * seed + b)
        target = torch.randn(b, 5, V, generator=g) * 2.0
        draft_logits = target[:, :4] + torch.randn(b, 4, V, generator=g) * 0.5
        p = osamp.probabilities(target, temperature)
        q = osamp.probabilities(draft_logits, temperature)
        draft = torch.multinomial(q.reshape(-1, V), 1, generator=g).view(b, 4)
        ua = torch.rand(b, 4, generator=g)
        ur = torch.rand(b, generator=g)
        want = oa.accept_reject(p, q, draft, u_accept=ua, u_residual=ur)
        # the kernel path from logits: device softmax, then the fused accept
        pd = probabilities(target.cuda(), temperature)
        qd = probabilities(draft_logits.cuda(), temperature)
        got = accept_reject(pd, qd, draft, u_accept=ua, u_residual=ur)
        near = oa.accept_reject_exclusion(p, q, draft, ua, ur)
        ok = (got.n_accepted == want.n_accepted) & (got.next_token == want.next_token)
        assert bool((ok | near).all()), (got, want, near)
        assert int(ok.sum()) >= b - 1


@pytest.mark.parametrize("vocab", [1001, 4099, 49151])
def test_fp32_rows_of_any_length_match_oracle(vocab):
    """fp32 rows whose length is not a multiple of 4 (the register-resident
    kernels then load 4 bytes at a time; elements past the row read as
    zero): accept-reject and the standalone inverse-CDF sampler against the
    oracle, bit-exact except rows decided within 1e-6 of a threshold."""
    b, k = 8, 4
    for seed in range(3):
        g = torch.Generator().manual_seed(vocab + seed)
        target = torch.randn(b, k + 1, vocab, generator=g) * 2.0
        draft_logits = target[:, :k] + torch.randn(b, k, vocab, generator=g) * 0.5
        p = osamp.probabilities(target, 1.0)
        q = osamp.probabilities(draft_logits, 1.0)
        draft = torch.multinomial(q.reshape(-1, vocab), 1, generator=g).view(b, k)
        ua, ur = torch.rand(b, k, generator=g), torch.rand(b, generator=g)
        want = oa.accept_reject(p, q, draft, u_accept=ua, u_residual=ur)
        got = accept_reject(p.cuda(), q.cuda(), draft, u_accept=ua, u_residual=ur)
        near = oa.accept_reject_exclusion(p, q, draft, ua, ur)
        ok = (got.n_accepted == want.n_accepted) & (got.next_token == want.next_token)
        assert bool((ok | near).all()), (vocab, seed, got, want, near)
        # the sampler alone on the target's bonus rows
        rows = p[:, k].contiguous()
        assert torch.equal(sample_inverse_cdf(rows.cuda(), ur).cpu(), oa.sample_inverse_cdf(rows, ur))


def test_config1_distribution_matches_target_softmax():
    """10,000 seeded rounds on config 1: the first emitted token's empirical
    distribution is the target softmax (chi-square GoF over tokens with
    expected count >= 5, the rest pooled)."""
    from scipy.stats import chisquare

    target, draft_logits = config1_logits(7)
    p = osamp.probabilities(target, 1.0)
    q = osamp.probabilities(draft_logits, 1.0)
    n = 10_000
    g = torch.Generator().manual_seed(8)
    draft = torch.multinomial(q, n, replacement=True, generator=g).T.contiguous()  # [n, 4]
    pd = p.cuda().unsqueeze(0).expand(n, 5, V)
    qd = q.cuda().unsqueeze(0).expand(n, 4, V)
    verdict = accept_reject(pd, qd, draft, generator=g)
    first = torch.where(verdict.n_accepted >= 1, draft[:, 0], verdict.next_token)
    counts = torch.bincount(first, minlength=V).double()
    expected = p[0].double() * n
    big = expected >= 5
    obs = torch.cat([counts[big], counts[~big].sum().view(1)])
    exp = torch.cat([expected[big], expected[~big].sum().view(1)])
    exp = exp * (obs.sum() / exp.sum())
    assert chisquare(obs.numpy(), exp.numpy()).pvalue > 1e-3


def test_custom_residual_is_used():
    """A residual callable replaces the fused residual (spec/accept.py:51)."""
    p = t64(P).expand(64, 2, 5)
    q = t64(Q).expand(64, 1, 5)
    draft = torch.full((64, 1), 2)
    ua = torch.full((64, 1), 0.9, dtype=torch.float64)  # always reject token 2 (ratio 2/3)
    ur = (torch.arange(64, dtype=torch.float64) + 0.5) / 64

    def argmax_of_residual(pp, qq):
        r = torch.clamp(pp - qq, min=0.0)
        return torch.nn.functional.one_hot(r.argmax(dim=-1), pp.shape[-1]).to(pp.dtype)

    got = accept_reject(p, q, draft, u_accept=ua, u_residual=ur, residual=argmax_of_residual)
    want = oa.accept_reject(p, q, draft, u_accept=ua, u_residual=ur, residual=argmax_of_residual)
    assert got.n_accepted.tolist() == want.n_accepted.tolist() == [0] * 64
    assert got.next_token.tolist() == want.next_token.tolist() == [0] * 64


def test_wrappers_reject_host_buffers_next_to_device_ones():
    """A host tensor among device inputs (or a short or mistyped one) raises
    on the host; nothing is launched with a host pointer."""
    from specdec import ops

    v = 64
    p = torch.rand(2, 5, v, device="cuda")
    q = torch.rand(2, 4, v, device="cuda")
    draft = torch.zeros(2, 4, dtype=torch.int64, device="cuda")
    ua = torch.rand(2, 4, device="cuda")
    with pytest.raises(RuntimeError, match="must be on"):
        ops.accept_reject(p, q, draft, ua, torch.rand(2))
    with pytest.raises(RuntimeError, match="must be on"):
        ops.accept_reject(p, q, draft.cpu(), ua, torch.rand(2, device="cuda"))
    with pytest.raises(ValueError, match="4 elements|8 elements"):
        ops.accept_count(p, q, draft, ua[:1])
    with pytest.raises(TypeError):
        ops.accept_count(p, q, draft.int(), ua)
    with pytest.raises(ValueError):
        ops.accept_count(p, q[:, :3], draft, ua)
    with pytest.raises(RuntimeError, match="must be on"):
        ops.probabilities(torch.randn(3, v, device="cuda"), 1.0, out=torch.empty(3, v))
    with pytest.raises(RuntimeError, match="must be on"):
        ops.ngram_lookup(torch.zeros(2, 8, dtype=torch.int32, device="cuda"), torch.full((2,), 8, dtype=torch.int32),
                         4, 3)
    torch.cuda.synchronize()
