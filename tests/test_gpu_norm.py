"""Layer glue kernels (residual add + RMSNorm, SiLU(gate) * up) against a
torch fp32 statement of transformers' Llama modules, at the decode sizes of
both models and at sizes that take the general kernels."""
import pytest
import torch

from specdec import ops

pytestmark = pytest.mark.gpu


def rmsnorm_ref(hidden, delta, weight, eps):
    """transformers' LlamaRMSNorm after the residual add, in the activation
    dtype: the add rounds, the norm runs in fp32 and rounds, then the weight."""
    h = hidden if delta is None else (hidden.float() + delta.float()).to(hidden.dtype)
    x = h.float()
    inv = torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + eps)
    return h, (weight.float() * (x * inv).to(hidden.dtype).float()).to(hidden.dtype)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize(("rows", "dim"), [(1, 576), (5, 2048), (3, 4096), (2, 100), (1, 8192), (7, 1536)])
@pytest.mark.parametrize("with_delta", [True, False])
def test_add_rmsnorm_matches_torch(dtype, rows, dim, with_delta):
    g = torch.Generator(device="cuda").manual_seed(rows * 7 + dim)
    hidden = torch.randn(rows, dim, generator=g, device="cuda").to(dtype)
    delta = torch.randn(rows, dim, generator=g, device="cuda").to(dtype) if with_delta else None
    weight = (1 + 0.1 * torch.randn(dim, generator=g, device="cuda")).to(dtype)
    want_h, want = rmsnorm_ref(hidden, delta, weight, 1e-5)
    h = hidden.clone()
    out = torch.empty_like(hidden)
    ops.add_rmsnorm(h, delta, weight, out, 1e-5)
    assert torch.equal(h, want_h)  # the residual add is exact
    # the sum of squares is reduced in another order than torch's, so the
    # row's scale can differ in its last bit: in fp32 every element then
    # moves by about an ulp, in bf16 an element rarely rounds the other way
    if dtype == torch.bfloat16:
        assert torch.allclose(out.float(), want.float(), rtol=2 ** -7, atol=1e-6)
        assert (out != want).float().mean().item() < 0.01
    else:
        assert torch.allclose(out, want, rtol=2e-6, atol=1e-7), (out - want).abs().max()


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize(("rows", "inter"), [(1, 1536), (5, 8192), (2, 100), (3, 12)])
def test_silu_mul_matches_torch(dtype, rows, inter):
    g = torch.Generator(device="cuda").manual_seed(rows + inter)
    gu = (3 * torch.randn(rows, 2 * inter, generator=g, device="cuda")).to(dtype)
    gate, up = gu[:, :inter].float(), gu[:, inter:].float()
    want = ((gate / (1 + torch.exp(-gate))).to(dtype).float() * up).to(dtype)
    out = torch.empty(rows, inter, dtype=dtype, device="cuda")
    ops.silu_mul(gu, out)
    if dtype == torch.bfloat16:
        assert torch.allclose(out.float(), want.float(), rtol=2 ** -7, atol=1e-6)
        assert (out != want).float().mean().item() < 0.01
    else:
        assert torch.allclose(out, want, rtol=2e-6, atol=1e-7), (out - want).abs().max()
