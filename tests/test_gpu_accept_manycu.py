"""The many-CU accept-reject kernel (each row spread over many workgroups of
one launch that exchange chunk values twice) against the one-workgroup-per-row
kernel and the oracle (spec/accept.py:44-79).  The two kernels add the
residual and the prefix sums in fp64 in different orders, so a row may
differ only where the oracle's 1e-6 exclusion band says the decision sits
on a threshold; elsewhere accept counts, tokens and flags agree exactly."""
import pytest
import torch

import oracle.accept as oa
from specdec import ops

pytestmark = pytest.mark.gpu


def inputs(b, k, v, seed, noise=0.5, temperature=1.0):
    g = torch.Generator().manual_seed(seed)
    tl = torch.randn(b, k + 1, v, generator=g) * 2.0
    dl = tl[:, :k] + torch.randn(b, k, v, generator=g) * noise
    p = torch.softmax(tl / temperature, -1)
    q = torch.softmax(dl / temperature, -1)
    draft = (torch.multinomial(q.reshape(-1, v), 1, generator=g).view(b, k) if k > 0
             else torch.zeros(b, 0, dtype=torch.int64))
    ua, ur = torch.rand(b, k, generator=g), torch.rand(b, generator=g)
    return p, q, draft, ua, ur


def both(p, q, draft, ua, ur):
    dev = [t.cuda().contiguous() for t in (p, q, draft, ua, ur)]
    many = ops.accept_reject(*dev).cpu()
    one = ops.accept_reject(*dev, single=True).cpu()
    return many, one


def agree(p, q, draft, ua, ur, many, one):
    band = oa.accept_reject_exclusion(p, q, draft, ua, ur)
    same = (many[0] == one[0]) & (many[1] == one[1]) & (many[2] == one[2])
    want = oa.accept_reject(p, q, draft, u_accept=ua, u_residual=ur)
    vs_oracle = (many[0] == want.n_accepted) & (many[1] == want.next_token)
    return bool((same | band).all()) and bool((vs_oracle | band).all()), int((~same).sum())


@pytest.mark.parametrize("v", [5, 17, 1000, 4099, 49152, 65536])
@pytest.mark.parametrize("b,k", [(1, 4), (2, 1), (5, 8), (8, 4), (16, 9), (32, 8), (64, 4), (3, 2)])
def test_many_cu_matches_single_and_oracle(v, b, k):
    p, q, draft, ua, ur = inputs(b, k, v, seed=v * 7 + b * 13 + k)
    many, one = both(p, q, draft, ua, ur)
    ok, differing = agree(p, q, draft, ua, ur, many, one)
    assert ok, (differing, many, one)
    assert bool((many[2] == 0).all())


def test_bonus_and_equal_distributions():
    """Every draft accepted (u = 0): the bonus token is sampled from p[k]; and
    p == q everywhere: the residual mass is zero and p itself is sampled."""
    b, k, v = 4, 4, 49152
    p, q, draft, ua, ur = inputs(b, k, v, seed=3)
    ua.zero_()
    many, one = both(p, q, draft, ua, ur)
    assert many[0].tolist() == [k] * b
    ok, _ = agree(p, q, draft, ua, ur, many, one)
    assert ok
    q_eq = p[:, :k].clone()
    draft_eq = torch.multinomial(q_eq.reshape(-1, v), 1, generator=torch.Generator().manual_seed(4)).view(b, k)
    ua = torch.full((b, k), 0.999)
    ua[:, 2] = 1.0  # u * q(x) < p(x) fails only where u = 1: n = 2 in every row
    many, one = both(p, q_eq, draft_eq, ua, ur)
    assert many[0].tolist() == [2] * b
    ok, _ = agree(p, q_eq, draft_eq, ua, ur, many, one)
    assert ok


def test_bad_draft_flag_and_out_of_range_ids():
    b, k, v = 3, 4, 4096
    p, q, draft, ua, ur = inputs(b, k, v, seed=5)
    q[1, 2, draft[1, 2]] = 0.0  # a zero draft probability
    draft[2, 1] = v  # an id outside the vocabulary
    many, one = both(p, q, draft, ua, ur)
    assert many[2].tolist() == one[2].tolist() == [0, 1, 1]
    assert many[0].tolist()[1:] == one[0].tolist()[1:]


def test_workspace_reused_across_shapes_stays_exact():
    """One workspace, calls of different batch and vocab back to back: the
    meeting words of earlier calls carry earlier tags and are never read as
    the current call's, so every call equals one on a fresh workspace, and
    the epoch counts the calls."""
    ws = ops.AcceptWorkspace(torch.device("cuda"))
    ws.reserve(64)  # sized once: a larger buffer would start a fresh epoch
    cases = [inputs(b, k, v, seed=s) for s, (b, k, v) in enumerate([(8, 4, 49152), (1, 4, 49152), (32, 8, 4099),
                                                                     (2, 2, 17), (64, 4, 49152)])]
    for rep in range(3):
        for i, (p, q, draft, ua, ur) in enumerate(cases):
            dev = [t.cuda().contiguous() for t in (p, q, draft, ua, ur)]
            got = ops.accept_reject(*dev, workspace=ws).cpu()
            fresh = ops.accept_reject(*dev, workspace=ops.AcceptWorkspace(torch.device("cuda"))).cpu()
            assert torch.equal(got, fresh), (rep, i)
    words = ws.buf.view(torch.int64)
    assert int(words[2]) == 3 * len(cases)  # the epoch
    assert int(words[(3 * len(cases)) % 2]) == 0  # the next call's arrival counter


@pytest.mark.parametrize("spin", [-1, 0])
@pytest.mark.parametrize("b,k,v", [(1, 4, 49152), (8, 4, 49152), (32, 8, 49152), (5, 8, 4099), (16, 9, 65536),
                                   (3, 2, 1000)])
def test_workgroups_that_stop_waiting_compute_the_same_bits(spin, b, k, v):
    """spin < 0: no workgroup waits for any other, each computes every other
    chunk's sums and prefixes itself; spin 0: one read, then the same for
    whatever is missing.  Every kernel exits normally and the output has the
    bits of the default, waiting path."""
    p, q, draft, ua, ur = inputs(b, k, v, seed=b * 31 + k + v)
    dev = [t.cuda().contiguous() for t in (p, q, draft, ua, ur)]
    want = ops.accept_reject(*dev).cpu()
    for rep in range(2):
        got = ops.accept_reject(*dev, spin=spin).cpu()
        assert torch.equal(got, want), (rep, got, want)
    # and the bad-draft flag survives the recomputing path
    q_bad = dev[1].clone()
    q_bad[0, 0, dev[2][0, 0]] = 0.0
    bad = ops.accept_reject(dev[0], q_bad, *dev[2:], spin=spin).cpu()
    assert int(bad[2, 0]) == 1
    assert torch.equal(bad, ops.accept_reject(dev[0], q_bad, *dev[2:]).cpu())


def test_graph_replays_match_eager():
    from lm.graphs import _capture

    p, q, draft, ua, ur = (t.cuda().contiguous() for t in inputs(1, 4, 49152, seed=9))
    ws = ops.AcceptWorkspace(torch.device("cuda"))
    ws.reserve(1)
    want = ops.accept_reject(p, q, draft, ua, ur, workspace=ws)
    out = torch.empty_like(want)
    graph, _ = _capture(lambda: out.copy_(ops.accept_reject(p, q, draft, ua, ur, workspace=ws)))
    for i in range(4):
        out.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, want), i
        assert torch.equal(ops.accept_reject(p, q, draft, ua, ur, workspace=ws), want), i
