"""Oracle of spec/accept.py (test infrastructure, see oracle/__init__.py)."""
from dataclasses import dataclass

import torch


def residual_distribution(p: torch.Tensor, q: torch.Tensor) -> torch.Tensor:
    """spec/accept.py:18-26: norm(max(0, p - q)), p where the mass is zero."""
    r = (p - q).clamp(min=0.0)
    total = r.sum(dim=-1, keepdim=True)
    return torch.where(total > 0, r / total.clamp(min=torch.finfo(r.dtype).tiny), p)


def sample_inverse_cdf(probs: torch.Tensor, u: torch.Tensor) -> torch.Tensor:
    """spec/accept.py:29-35: searchsorted(right) of u*total in the cumsum."""
    cdf = probs.cumsum(dim=-1)
    target = (u * cdf[:, -1]).unsqueeze(-1)
    return torch.searchsorted(cdf, target, right=True).squeeze(-1).clamp(max=probs.shape[-1] - 1)


@dataclass(frozen=True)
class Verdict:
    """spec/accept.py:38-41"""
    n_accepted: torch.Tensor
    next_token: torch.Tensor


def accept_reject(p, q, draft, generator=None, u_accept=None, u_residual=None, residual=residual_distribution):
    """spec/accept.py:44-79, on the CPU."""
    b, k = draft.shape
    if u_accept is None:
        u_accept = torch.rand(b, k, generator=generator, dtype=p.dtype, device=p.device)
    if u_residual is None:
        u_residual = torch.rand(b, generator=generator, dtype=p.dtype, device=p.device)
    idx = draft.unsqueeze(-1)
    p_x = p[:, :k].gather(-1, idx).squeeze(-1)
    q_x = q.gather(-1, idx).squeeze(-1)
    if not bool((q_x > 0).all()):
        raise ValueError("a drafted token has zero draft probability; q is not what it was sampled from")
    accepted = u_accept * q_x < p_x
    n_accepted = accepted.long().cumprod(dim=-1).sum(dim=-1)
    q_padded = torch.cat([q, torch.zeros_like(q[:, :1])], dim=1)
    rows = torch.arange(b, device=p.device)
    r = residual(p[rows, n_accepted], q_padded[rows, n_accepted])
    return Verdict(n_accepted, sample_inverse_cdf(r, u_residual))


def accept_reject_exclusion(p, q, draft, u_accept, u_residual, band: float = 1e-6):
    """Which rows of an oracle verdict are decided within `band` of a
    threshold: the accept test |u - p/q| < band at any tested position, or
    the sampled token's CDF interval boundary within band * total of the
    target.  Rows flagged here may legitimately differ between two correct
    implementations whose fp32 sums round differently."""
    b, k = draft.shape
    idx = draft.unsqueeze(-1)
    p_x = p[:, :k].gather(-1, idx).squeeze(-1).double()
    q_x = q.gather(-1, idx).squeeze(-1).double()
    near = ((u_accept.double() - p_x / q_x).abs() < band).any(dim=-1)
    verdict = accept_reject(p, q, draft, u_accept=u_accept, u_residual=u_residual)
    q_padded = torch.cat([q, torch.zeros_like(q[:, :1])], dim=1)
    rows = torch.arange(b)
    r = residual_distribution(p[rows, verdict.n_accepted], q_padded[rows, verdict.n_accepted]).double()
    cdf = r.cumsum(-1)
    target = u_residual.double() * cdf[:, -1]
    dist = (cdf - target[:, None]).abs().min(dim=-1).values
    near |= dist < band * cdf[:, -1]
    return near
