"""Pins oracle.accept: the reference's known answers, golden vectors written
by the reference itself, a closed form and a statistical check."""
from fractions import Fraction

import pytest
import torch

import oracle.accept as oa
from helpers import golden
from workloads import accept_inputs

P = [Fraction(4, 10), Fraction(3, 10), Fraction(2, 10), Fraction(1, 10), Fraction(0)]
Q = [Fraction(1, 10), Fraction(2, 10), Fraction(3, 10), Fraction(1, 10), Fraction(3, 10)]
ACCEPT = [Fraction(1), Fraction(1), Fraction(2, 3), Fraction(1), Fraction(0)]


def t64(xs):
    return torch.tensor([float(x) for x in xs], dtype=torch.float64)


def test_rejection_mass_is_one_minus_overlap():
    """The probability of rejecting the draft, sum(max(0, p - q)), and the
    overlap sum(min(p, q)) of the toy pair add up to one (exact fractions)."""
    beta = sum(max(Fraction(0), p - q) for p, q in zip(P, Q))
    overlap = sum(min(p, q) for p, q in zip(P, Q))
    assert beta == Fraction(2, 5) and beta + overlap == 1
    # the accept probabilities of the toy pair weigh q to the same overlap
    assert sum(q * a for q, a in zip(Q, ACCEPT)) == overlap


def test_residual_hand_values():
    r = oa.residual_distribution(t64(P), t64(Q))
    assert torch.allclose(r, t64([Fraction(3, 4), Fraction(1, 4), 0, 0, 0]), atol=1e-15, rtol=0)


def test_residual_of_equal_distributions_falls_back_to_p():
    p = torch.tensor([[0.25, 0.75]], dtype=torch.float64)
    assert torch.equal(oa.residual_distribution(p, p), p)


def test_coupled_grid_exact_fractions():
    n = 120
    grid = (torch.arange(n, dtype=torch.float64) + 0.5) / n
    ua, ur = grid.repeat_interleave(n).unsqueeze(-1), grid.repeat(n)
    p, q = t64(P).expand(n * n, 2, 5), t64(Q).expand(n * n, 1, 5)
    emitted = [Fraction(0)] * 5
    for y in range(5):
        draft = torch.full((n * n, 1), y)
        v = oa.accept_reject(p, q, draft, u_accept=ua, u_residual=ur)
        first = torch.where(v.n_accepted == 1, draft[:, 0], v.next_token)
        assert Fraction(int(v.n_accepted.sum()), n * n) == ACCEPT[y]
        for x, c in enumerate(torch.bincount(first, minlength=5).tolist()):
            emitted[x] += Q[y] * Fraction(c, n * n)
    assert emitted == P


def test_scripted_and_greedy_known_answers():
    p, q, d = t64(P).expand(1, 2, 5), t64(Q).expand(1, 1, 5), torch.tensor([[2]])
    run = lambda ua, ur: oa.accept_reject(p, q, d, u_accept=torch.tensor([[ua]], dtype=torch.float64),
                                          u_residual=torch.tensor([ur], dtype=torch.float64))
    assert (run(0.6, 0.5).n_accepted.item(), run(0.6, 0.5).next_token.item()) == (1, 1)
    assert (run(0.7, 0.8).n_accepted.item(), run(0.7, 0.8).next_token.item()) == (0, 1)
    assert run(0.7, 0.5).next_token.item() == 0
    ph = torch.nn.functional.one_hot(torch.tensor([[3, 1, 4]]), 5).double()
    v = oa.accept_reject(ph, torch.nn.functional.one_hot(torch.tensor([[3, 2]]), 5).double(), torch.tensor([[3, 2]]),
                         generator=torch.Generator().manual_seed(0))
    assert (v.n_accepted.item(), v.next_token.item()) == (1, 1)


def test_inverse_cdf_equals_brute_force_interval_search():
    """searchsorted(right) of u*total == the unique i with cdf[i-1] <= u*total < cdf[i]."""
    g = torch.Generator().manual_seed(0)
    probs = torch.rand(50, 9, generator=g, dtype=torch.float64)
    probs[probs < 0.3] = 0
    probs[:, 0] += 1e-3
    u = torch.rand(50, generator=g, dtype=torch.float64)
    got = oa.sample_inverse_cdf(probs, u)
    for row in range(50):
        cdf = probs[row].cumsum(0)
        target = u[row] * cdf[-1]
        want = next(i for i in range(9) if target < cdf[i])
        assert got[row].item() == want
        assert probs[row, want] > 0


def test_cumsum_accumulates_in_fp64_per_prefix():
    """CPU fp32 cumsum rounds an fp64 running sum once per prefix; the kernels
    follow that rule, so pin it here."""
    x = torch.softmax(torch.randn(49152, generator=torch.Generator().manual_seed(1)) * 2, -1)
    acc, ref = 0.0, []
    for v in x.double().tolist():
        acc += v
        ref.append(acc)
    assert torch.equal(x.cumsum(0), torch.tensor(ref, dtype=torch.float64).float())


@pytest.mark.parametrize("i", range(4))
def test_golden_generator_stream(i):
    case = golden("accept_gen.json")["cases"][i]
    dtype = getattr(torch, case["dtype"])
    if case["p"] is not None:
        p, q, draft = torch.tensor(case["p"], dtype=dtype), torch.tensor(case["q"], dtype=dtype), torch.tensor(case["draft"])
    else:
        p, q, draft = accept_inputs(dtype, case["b"], case["k"], case["v"], case["noise"], case["input_seed"])
    import hashlib

    assert hashlib.sha256(p.numpy().tobytes()).hexdigest() == case["p_sha"]
    v = oa.accept_reject(p, q, draft, generator=torch.Generator().manual_seed(case["seed"]))
    assert v.n_accepted.tolist() == case["n_accepted"] and v.next_token.tolist() == case["next_token"]
    # the uniforms are u_accept [B, k] then u_residual [B] in p's dtype
    gu = torch.Generator().manual_seed(case["seed"])
    assert torch.rand(case["b"], case["k"], generator=gu, dtype=dtype).tolist() == case["u_accept"]
    assert torch.rand(case["b"], generator=gu, dtype=dtype).tolist() == case["u_residual"]


def test_output_distribution_is_p_and_broken_residual_is_caught():
    from scipy.stats import chisquare

    torch.manual_seed(0)
    d = torch.distributions.Dirichlet(torch.ones(16, dtype=torch.float64))
    p, q = d.sample(), d.sample()
    n = 40_000
    g = torch.Generator().manual_seed(2)
    draft = torch.multinomial(q, n * 2, replacement=True, generator=g).view(n, 2)
    for residual, good in [(oa.residual_distribution, True), (lambda pp, qq: pp, False)]:
        gg = torch.Generator().manual_seed(3)
        v = oa.accept_reject(p.expand(n, 3, 16), q.expand(n, 2, 16), draft, generator=gg, residual=residual)
        first = torch.where(v.n_accepted >= 1, draft[:, 0], v.next_token)
        counts = torch.bincount(first, minlength=16).double()
        pv = chisquare(counts.numpy(), (p * n).numpy()).pvalue
        assert (pv > 1e-3) == good
