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


def host_draft(verdict: Verdict) -> torch.Tensor | None:
    """The [B, k] host copy of the draft that came back in the verdict's
    device-to-host copy, or None.  It is an attribute outside the dataclass's
    fields, so `fields`, `astuple`, `==` and `repr` of a Verdict are those of
    the reference's two-field type (spec/accept.py:38-41)."""
    return getattr(verdict, "_host_draft", None)


_BAD_DRAFT = ("a drafted token has zero draft probability or lies outside the vocabulary; q is not what it "
              "was sampled from")


def _settle(out: torch.Tensor, draft_d: torch.Tensor) -> Verdict:
    """The kernel's [3, B] output and the draft brought to the host in one
    copy; the reference's ValueError for a bad draft."""
    host = torch.cat([out, draft_d.t()]).cpu()
    if bool(host[2].any()):
        raise ValueError(_BAD_DRAFT)
    verdict = Verdict(host[0].clone(), host[1].clone())
    object.__setattr__(verdict, "_host_draft", host[3:].t())
    return verdict


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
        return _settle(ops.accept_reject(p, q, draft_d, ua, ur), draft_d)
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


def accept_reject_logits(
    target_logits: torch.Tensor,
    draft_logits: torch.Tensor,
    draft: torch.Tensor,
    temperature: float,
    generator: torch.Generator | None = None,
    u_accept: torch.Tensor | None = None,
    u_residual: torch.Tensor | None = None,
) -> Verdict:
    """accept_reject(probabilities(target_logits, T), probabilities(draft_logits, T), draft, ...)
    with p and q never materialised: target_logits [B, k+1, V] and
    draft_logits [B, k, V] (lm/sampling.py:13-18 then spec/accept.py:44-79).
    One launch reads each logit once and returns the same verdict the two
    steps give (up to the last bits of the softmax, as two softmax kernels
    differ).  Uniforms are drawn as accept_reject draws them (fp32, u_accept
    then u_residual).  Shapes the fused kernel does not take run the two
    steps."""
    b, k = draft.shape
    if u_accept is None:
        u_accept = _uniforms((b, k), generator, torch.float32)
    if u_residual is None:
        u_residual = _uniforms((b,), generator, torch.float32)
    tl = _cuda(target_logits).float()
    dl = _cuda(draft_logits).float()
    draft_d = _cuda(draft.to(torch.int64)).contiguous()
    ua = _cuda(u_accept.float()).contiguous()
    ur = _cuda(u_residual.float()).contiguous()
    out = ops.accept_reject_logits(tl, dl, temperature, draft_d, ua, ur)
    if out is None:
        from lm.sampling import probabilities

        return accept_reject(probabilities(tl, temperature), probabilities(dl, temperature), draft, u_accept=ua,
                             u_residual=ur)
    return _settle(out, draft_d)
