"""Accept-reject from logits in one launch (specdec_accept_reject_logits):
probabilities() of the target and draft logits (lm/sampling.py:13-18)
followed by accept_reject (spec/accept.py:44-79), with p and q formed inside
the launch from row statistics.

Checked against the oracle -- torch's CPU softmax, then the reference's
accept-reject -- on the same logits and uniforms: accept counts and tokens
bit-exact except rows the oracle's 1e-6 exclusion band flags (two correct
softmax implementations differ in the last bits, and a decision within 1e-6
of its threshold may go either way).  Against the two-launch GPU path
(softmax kernel, then the many-CU accept) the same.  Greedy (T = 0) rows
have no band: one-hot rows are exact."""
import pytest
import torch

import oracle.accept as oa
import oracle.sampling as osamp
from spec.accept import Verdict, accept_reject, accept_reject_logits
from specdec import ops

pytestmark = pytest.mark.gpu
V = 49152


def logits(b, k, v, seed, noise=0.5, scale=2.0):
    g = torch.Generator().manual_seed(seed)
    tl = torch.randn(b, k + 1, v, generator=g) * scale
    dl = tl[:, :k] + torch.randn(b, k, v, generator=g) * noise
    return tl, dl, g


def drafts_from(dl, temperature, g):
    b, k, v = dl.shape
    q = osamp.probabilities(dl, temperature)
    return torch.multinomial(q.reshape(-1, v), 1, generator=g).view(b, k)


def fused(tl, dl, temperature, draft, ua, ur, spin=ops.ACCEPT_SPIN):
    out = ops.accept_reject_logits(tl.cuda(), dl.cuda(), temperature, draft.cuda(), ua.cuda(), ur.cuda(), spin=spin)
    assert out is not None, "the shape should take the fused kernel"
    return out.cpu()


def check_vs_oracle(tl, dl, temperature, draft, ua, ur, got):
    p = osamp.probabilities(tl, temperature)
    q = osamp.probabilities(dl, temperature)
    want = oa.accept_reject(p, q, draft, u_accept=ua, u_residual=ur)
    ok = (got[0] == want.n_accepted) & (got[1] == want.next_token)
    if temperature == 0.0:
        assert bool(ok.all()), (got, want)
    else:
        near = oa.accept_reject_exclusion(p, q, draft, ua, ur)
        assert bool((ok | near).all()), (got, want, near)
        assert int(ok.sum()) >= got.shape[1] - max(1, got.shape[1] // 8)
    assert bool((got[2] == 0).all())


@pytest.mark.parametrize("seed", range(4))
@pytest.mark.parametrize("b,k,temperature", [(1, 4, 1.0), (1, 4, 0.8), (8, 4, 1.0), (8, 8, 0.8), (32, 8, 0.8),
                                             (32, 4, 1.0), (3, 2, 1.3), (1, 1, 1.0), (2, 16, 0.8), (16, 4, 0.8),
                                             (24, 8, 1.0), (48, 8, 0.8), (64, 4, 1.0)])
def test_fused_matches_oracle(seed, b, k, temperature):
    tl, dl, g = logits(b, k, V, seed=seed * 101 + b * 7 + k)
    draft = drafts_from(dl, temperature, g)
    ua, ur = torch.rand(b, k, generator=g), torch.rand(b, generator=g)
    check_vs_oracle(tl, dl, temperature, draft, ua, ur, fused(tl, dl, temperature, draft, ua, ur))


@pytest.mark.parametrize("b,k,v,temperature", [(1, 4, 4100, 1.0), (2, 4, 40004, 0.8), (3, 3, 1000, 1.3),
                                               (8, 2, 50000, 0.0), (24, 8, 12, 0.8)])
def test_ragged_last_chunk_matches_oracle(b, k, v, temperature):
    """Vocabularies that are not a multiple of a chunk (and one smaller than
    a thread's elements): the last chunk's missing elements take no part in
    any row's max, sum, residual or prefix."""
    tl, dl, g = logits(b, k, v, seed=v + b)
    draft = drafts_from(dl, temperature, g) if temperature > 0 else dl.argmax(-1)
    ua, ur = torch.rand(b, k, generator=g), torch.rand(b, generator=g)
    check_vs_oracle(tl, dl, temperature, draft, ua, ur, fused(tl, dl, temperature, draft, ua, ur))


@pytest.mark.parametrize("b,k", [(1, 4), (8, 4), (32, 8)])
def test_greedy_is_argmax_verification(b, k):
    """T = 0: p and q are one-hot rows of the argmax (lowest id among ties);
    drafting the draft's argmax, the accepted prefix is where the target's
    argmax agrees and the next token is the target's argmax there."""
    tl, dl, g = logits(b, k, V, seed=b + k, noise=2.0)
    tl[0, 0, 7] = tl[0, 0, 3] = tl[0, 0].max() + 1.0  # a tie: id 3 wins
    draft = dl.argmax(-1)
    ua, ur = torch.rand(b, k, generator=g), torch.rand(b, generator=g)
    got = fused(tl, dl, 0.0, draft, ua, ur)
    check_vs_oracle(tl, dl, 0.0, draft, ua, ur, got)
    targ = tl.argmax(-1)
    for r in range(b):
        n = 0
        while n < k and int(draft[r, n]) == int(targ[r, n]):
            n += 1
        assert int(got[0, r]) == n and int(got[1, r]) == int(targ[r, n])


@pytest.mark.parametrize("b,k,temperature", [(1, 4, 1.0), (8, 4, 0.8), (32, 8, 0.8), (48, 8, 1.0)])
def test_fused_matches_two_launch_gpu_path(b, k, temperature):
    """The same decisions as the softmax kernel followed by the many-CU
    accept kernel, except rows decided within 1e-6 of a threshold."""
    for seed in range(3):
        tl, dl, g = logits(b, k, V, seed=1000 + seed)
        draft = drafts_from(dl, temperature, g)
        ua, ur = torch.rand(b, k, generator=g), torch.rand(b, generator=g)
        got = fused(tl, dl, temperature, draft, ua, ur)
        pd = ops.probabilities(tl.cuda(), temperature)
        qd = ops.probabilities(dl.cuda(), temperature)
        two = ops.accept_reject(pd, qd, draft.cuda(), ua.cuda(), ur.cuda()).cpu()
        near = oa.accept_reject_exclusion(pd.cpu(), qd.cpu(), draft, ua, ur)
        same = (got[0] == two[0]) & (got[1] == two[1]) & (got[2] == two[2])
        assert bool((same | near).all()), (got, two)


@pytest.mark.parametrize("spin", [-1, 0])
@pytest.mark.parametrize("b,k,temperature,v", [(1, 4, 1.0, V), (8, 8, 0.8, V), (32, 8, 0.8, V), (4, 4, 0.0, V),
                                               (16, 4, 0.8, V), (64, 4, 0.8, V), (3, 4, 0.8, 40004)])
def test_workgroups_that_stop_waiting_compute_the_same_bits(spin, b, k, temperature, v):
    """No workgroup waits (spin < 0), or each reads once (spin 0): every
    missing chunk's statistics, sums and prefixes are computed by the reader
    with the code of the chunk's own workgroup, so the output has the bits
    of the waiting path."""
    tl, dl, g = logits(b, k, v, seed=77 + b)
    draft = drafts_from(dl, temperature, g) if temperature > 0 else dl.argmax(-1)
    ua, ur = torch.rand(b, k, generator=g), torch.rand(b, generator=g)
    want = fused(tl, dl, temperature, draft, ua, ur)
    for rep in range(2):
        assert torch.equal(fused(tl, dl, temperature, draft, ua, ur, spin=spin), want), rep


def test_bad_drafts_flagged():
    """A draft id outside the vocabulary, and (T = 0) a drafted token that is
    not the draft's argmax (q(x) = 0): flag 1, and spec.accept raises the
    reference's ValueError."""
    b, k = 3, 4
    tl, dl, g = logits(b, k, V, seed=5)
    ua, ur = torch.rand(b, k, generator=g), torch.rand(b, generator=g)
    draft = drafts_from(dl, 1.0, g)
    draft[2, 1] = V
    got = fused(tl, dl, 1.0, draft, ua, ur)
    assert got[2].tolist() == [0, 0, 1] and int(got[0, 2]) <= 1
    greedy = dl.argmax(-1)
    greedy[1, 0] = (greedy[1, 0] + 1) % V
    got = fused(tl, dl, 0.0, greedy, ua, ur)
    assert got[2].tolist() == [0, 1, 0]
    with pytest.raises(ValueError):
        accept_reject_logits(tl, dl, greedy, 0.0, u_accept=ua, u_residual=ur)


def test_every_draft_accepted_samples_the_bonus_row():
    b, k = 4, 4
    tl, dl, g = logits(b, k, V, seed=11)
    draft = drafts_from(dl, 1.0, g)
    ua, ur = torch.zeros(b, k), torch.rand(b, generator=g)
    got = fused(tl, dl, 1.0, draft, ua, ur)
    assert got[0].tolist() == [k] * b
    check_vs_oracle(tl, dl, 1.0, draft, ua, ur, got)


def test_api_draws_uniforms_like_accept_reject():
    """spec.accept.accept_reject_logits with a generator draws u_accept then
    u_residual as accept_reject does, and returns the reference's two-field
    Verdict with the same decisions as probabilities() + accept_reject."""
    b, k = 8, 4
    tl, dl, g = logits(b, k, V, seed=21)
    draft = drafts_from(dl, 0.8, g)
    got = accept_reject_logits(tl, dl, draft, 0.8, generator=torch.Generator().manual_seed(3))
    assert isinstance(got, Verdict)
    gen = torch.Generator().manual_seed(3)
    ua, ur = torch.rand(b, k, generator=gen), torch.rand(b, generator=gen)
    p, q = osamp.probabilities(tl, 0.8), osamp.probabilities(dl, 0.8)
    two = accept_reject(p.cuda(), q.cuda(), draft, u_accept=ua, u_residual=ur)
    near = oa.accept_reject_exclusion(p, q, draft, ua, ur)
    same = (got.n_accepted == two.n_accepted) & (got.next_token == two.next_token)
    assert bool((same | near).all())


def test_config1_distribution_matches_target_softmax():
    """10,000 seeded rounds of config 1 through the fused kernel (64 rounds
    per launch): the first emitted token's empirical distribution is the
    target softmax (chi-square GoF, tokens with expected count < 5 pooled)."""
    from scipy.stats import chisquare

    g = torch.Generator().manual_seed(7)
    target = torch.randn(5, V, generator=g) * 2.0
    draft_logits = target[:4] + torch.randn(4, V, generator=g) * 0.5
    p = osamp.probabilities(target, 1.0)
    q = osamp.probabilities(draft_logits, 1.0)
    n, per = 10_000, 64
    g = torch.Generator().manual_seed(8)
    draft = torch.multinomial(q, n, replacement=True, generator=g).T.contiguous()  # [n, 4]
    ua, ur = torch.rand(n, 4, generator=g), torch.rand(n, generator=g)
    tl = target.cuda().unsqueeze(0)
    dl = draft_logits.cuda().unsqueeze(0)
    first = []
    for r0 in range(0, n, per):
        r1 = min(n, r0 + per)
        m = r1 - r0
        out = ops.accept_reject_logits(tl.expand(m, 5, V), dl.expand(m, 4, V), 1.0, draft[r0:r1].cuda(),
                                       ua[r0:r1].cuda(), ur[r0:r1].cuda())
        assert out is not None
        out = out.cpu()
        first.append(torch.where(out[0] >= 1, draft[r0:r1, 0], out[1]))
    counts = torch.bincount(torch.cat(first), minlength=V).double()
    expected = p[0].double() * n
    big = expected >= 5
    obs = torch.cat([counts[big], counts[~big].sum().view(1)])
    exp = torch.cat([expected[big], expected[~big].sum().view(1)])
    exp = exp * (obs.sum() / exp.sum())
    assert chisquare(obs.numpy(), exp.numpy()).pvalue > 1e-3


@pytest.mark.parametrize("b,k,v", [(2, 17, 4096), (65, 2, V), (2, 4, 4099)])
def test_shapes_the_kernel_does_not_take_run_two_steps(b, k, v):
    """More than 16 drafted positions, more rows than two workgroups per
    compute unit hold (65 rows of a 49152 vocabulary), or rows that are not
    16-byte aligned (a vocabulary of 4099): the wrapper says so (None) and
    the API runs probabilities + accept_reject instead, with the same
    decisions."""
    tl, dl, g = logits(b, k, v, seed=2)
    draft = drafts_from(dl, 1.0, g)
    ua, ur = torch.rand(b, k, generator=g), torch.rand(b, generator=g)
    assert ops.accept_reject_logits(tl.cuda(), dl.cuda(), 1.0, draft.cuda(), ua.cuda(), ur.cuda()) is None
    got = accept_reject_logits(tl, dl, draft, 1.0, u_accept=ua, u_residual=ur)
    p, q = osamp.probabilities(tl, 1.0), osamp.probabilities(dl, 1.0)
    want = oa.accept_reject(p, q, draft, u_accept=ua, u_residual=ur)
    near = oa.accept_reject_exclusion(p, q, draft, ua, ur)
    same = (got.n_accepted == want.n_accepted) & (got.next_token == want.next_token)
    assert bool((same | near).all())


def test_graph_replays_match_eager():
    from lm.graphs import _capture

    tl, dl, g = logits(1, 4, V, seed=9)
    draft = drafts_from(dl, 1.0, g)
    ua, ur = torch.rand(1, 4, generator=g), torch.rand(1, generator=g)
    args = [t.cuda().contiguous() for t in (tl, dl)] + [1.0] + [t.cuda().contiguous() for t in (draft, ua, ur)]
    ws = ops.AcceptWorkspace(torch.device("cuda"))
    ws.reserve(1)
    want = ops.accept_reject_logits(*args, workspace=ws)
    out = torch.empty_like(want)
    graph, _ = _capture(lambda: out.copy_(ops.accept_reject_logits(*args, workspace=ws)))
    for i in range(4):
        out.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, want), i
        assert torch.equal(ops.accept_reject_logits(*args, workspace=ws), want), i
