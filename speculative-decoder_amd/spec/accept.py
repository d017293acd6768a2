"""Speculative-sampling accept-reject on the GPU (reference: spec/accept.py).

For drafted x ~ q, accepting with probability min(1, p(x)/q(x)) emits x with
probability min(p(x), q(x)); on rejection the residual norm(max(0, p - q))
supplies the missing mass max(0, p(x) - q(x)), so every emitted token is
distributed as p whatever q is.  The bonus position is the same residual
sample against an all-zero q row.

With the default residual the whole decision is one kernel launch
(specdec_accept_reject): gather p(x), q(x), the u*q(x) < p(x) test, the
leading-accept count, the residual and its inverse-CDF sample.  A custom
`residual` callable (used by the statistical tests to plant known bugs) is
evaluated by torch on the device between the accept kernel and the
inverse-CDF kernel.

Uniforms are drawn from the caller's generator in the reference's order and
dtype (u_accept [B, k], then u_residual [B]; spec/accept.py:60-63), on the
generator's device (the CPU for the loop's generator), then copied over.
"""
from __future__ import annotations

from collections.abc import Callable
from dataclasses import dataclass

import torch

from specdec import ops

Residual = Callable[[torch.Tensor, torch.Tensor], torch.Tensor]


def _cuda(x: torch.Tensor) -> torch.Tensor:
    return x if x.device.type == "cuda" else x.to("cuda", non_blocking=True)


def residual_distribution(p: torch.Tensor, q: torch.Tensor) -> torch.Tensor:
    """norm(max(0, p - q)) over the last dim (spec/accept.py:18-26), on the GPU.
    If the residual mass is zero (p == q) it falls back to p, which is never
    sampled in that case since no rejection can happen."""
    p, q = _cuda(p), _cuda(q)
    r = torch.clamp(p - q, min=0.0)
    total = r.sum(dim=-1, keepdim=True)
    return torch.where(total > 0, r / total.clamp(min=torch.finfo(r.dtype).tiny), p)


def sample_inverse_cdf(probs: torch.Tensor, u: torch.Tensor) -> torch.Tensor:
    """probs [B, V] (need not sum to 1), u [B] in [0, 1) -> token ids [B] on the
    GPU.  Token i is chosen iff u * total lies in [cdf[i-1], cdf[i]), with the
    prefix sums accumulated in fp64, so zero-probability tokens are never
    chosen (spec/accept.py:29-35)."""
    probs = _cuda(probs)
    u = _cuda(u.to(probs.dtype))
    return ops.sample_inverse_cdf(probs, u)


@dataclass(frozen=True)
class Verdict:
    n_accepted: torch.Tensor  # [B] leading draft tokens kept, 0..k
    next_token: torch.Tensor  # [B] residual sample at the first rejection, or the bonus token
    draft: torch.Tensor | None = None  # [B, k] host copy of the draft, brought back with the verdict


_BAD_DRAFT = ("a drafted token has zero draft probability or lies outside the vocabulary; q is not what it "
              "was sampled from")


def _uniforms(shape: tuple[int, ...], generator: torch.Generator | None, dtype: torch.dtype) -> torch.Tensor:
    device = generator.device if generator is not None else torch.device("cpu")
    return torch.rand(*shape, generator=generator, dtype=dtype, device=device)


def accept_reject(
    p: torch.Tensor,
    q: torch.Tensor,
    draft: torch.Tensor,
    generator: torch.Generator | None = None,
    u_accept: torch.Tensor | None = None,
    u_residual: torch.Tensor | None = None,
    residual: Residual = residual_distribution,
) -> Verdict:
    """p [B, k+1, V] target probabilities at each drafted position plus the
    bonus position, q [B, k, V] the draft distributions the tokens were
    sampled from, draft [B, k].  Returns the Verdict with host (CPU) int64
    tensors: the loop reads them element by element.

    Raises ValueError if a drafted token has zero draft probability (or is
    not a token id of the vocabulary)."""
    b, k = draft.shape
    if u_accept is None:
        u_accept = _uniforms((b, k), generator, p.dtype)
    if u_residual is None:
        u_residual = _uniforms((b,), generator, p.dtype)
    p = _cuda(p)
    q = _cuda(q.to(p.dtype))
    draft_d = _cuda(draft.to(torch.int64)).contiguous()
    ua = _cuda(u_accept.to(p.dtype)).contiguous()
    ur = _cuda(u_residual.to(p.dtype)).contiguous()
    if residual is residual_distribution:
        # the draft rides in the verdict's one copy to the host
        out = torch.cat([ops.accept_reject(p, q, draft_d, ua, ur), draft_d.t()]).cpu()
        ops.check_accept_flags(out[2], p.device)
        if bool(out[2].any()):
            raise ValueError(_BAD_DRAFT)
        return Verdict(out[0].clone(), out[1].clone(), out[3:].t())
    stage = ops.accept_count(p, q, draft_d, ua)
    n_host = stage.cpu()
    if bool(n_host[1].any()):
        raise ValueError(_BAD_DRAFT)
    n = stage[0]
    rows = torch.arange(b, device=p.device)
    q_padded = torch.cat([q, torch.zeros_like(q[:, :1])], dim=1)
    r = residual(p[rows, n], q_padded[rows, n])
    tokens = ops.sample_inverse_cdf(_cuda(r).to(p.dtype).contiguous(), ur)
    return Verdict(n_host[0].clone(), tokens.cpu())
