"""A seeded sweep of accept-reject call shapes against the oracle: 1-40 rows,
1-16 drafted positions, vocabularies from 7 to 65536 (multiples of 4 and
not), temperatures 0-1.7, draft noise from a near copy of the target to an
unrelated draft.  Every form runs on the same inputs: the many-CU kernel and
the one-workgroup kernel from probabilities, and the logits form where it
takes the shape.  Bit-exact tokens and accept counts except rows the
oracle's 1e-6 exclusion band flags (greedy rows have none)."""
import random

import pytest
import torch

import oracle.accept as oa
import oracle.sampling as osamp
from specdec import ops
from test_gpu_accept_logits import check_vs_oracle

pytestmark = pytest.mark.gpu


def _cases(n=40, seed=31):
    rng = random.Random(seed)
    out = []
    for i in range(n):
        b = rng.choice([1, 1, 2, 3, 8, 13, 32, 40])
        k = rng.choice([1, 2, 4, 4, 8, 16])
        v = rng.choice([7, 100, 1001, 4096, 4099, 33333, 49152, 49152, 65536])
        t = rng.choice([0.0, 0.5, 0.8, 1.0, 1.0, 1.7])
        noise = rng.choice([0.0, 0.05, 0.5, 3.0])
        out.append(pytest.param(b, k, v, t, noise, 500 + i, id=f"{i}-b{b}-k{k}-v{v}-t{t}-n{noise}"))
    return out


@pytest.mark.parametrize("b,k,v,temperature,noise,seed", _cases())
def test_random_shapes_every_form_matches_oracle(b, k, v, temperature, noise, seed):
    g = torch.Generator().manual_seed(seed)
    tl = torch.randn(b, k + 1, v, generator=g) * 2.0
    dl = tl[:, :k] + torch.randn(b, k, v, generator=g) * noise if noise > 0 else tl[:, :k].clone()
    p, q = osamp.probabilities(tl, temperature), osamp.probabilities(dl, temperature)
    if temperature > 0:
        draft = torch.multinomial(q.reshape(-1, v), 1, generator=g).view(b, k)
    else:
        draft = dl.argmax(-1)
    ua, ur = torch.rand(b, k, generator=g), torch.rand(b, generator=g)
    args = (draft.cuda(), ua.cuda(), ur.cuda())
    forms = {"many-CU": ops.accept_reject(p.cuda(), q.cuda(), *args),
             "one workgroup": ops.accept_reject(p.cuda(), q.cuda(), *args, single=True)}
    fused = ops.accept_reject_logits(tl.cuda(), dl.cuda(), temperature, *args)  # None: a shape it does not take
    if v % 4 == 0 and v <= 49152 and b <= 32:  # within its documented limit (64 rows of 49152)
        assert fused is not None
    if fused is not None:
        forms["logits"] = fused
    for name, got in forms.items():
        got = got.cpu()
        if name == "logits":
            check_vs_oracle(tl, dl, temperature, draft, ua, ur, got)
            continue
        want = oa.accept_reject(p, q, draft, u_accept=ua, u_residual=ur)
        ok = (got[0] == want.n_accepted) & (got[1] == want.next_token)
        near = oa.accept_reject_exclusion(p, q, draft, ua, ur) if temperature > 0 else torch.zeros_like(ok)
        assert bool((ok | near).all()), (name, got, want, near)
        assert bool((got[2] == 0).all()), name
