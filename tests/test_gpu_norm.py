"""Layer glue kernels (residual add + RMSNorm, SiLU(gate) * up, and SiLU * up
after a projection of the unnormalised stream) against a torch fp32
statement of transformers' Llama modules, at the decode sizes of both
models and at sizes that take the general kernels."""
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


def rms_silu_ref(gu, hidden, eps):
    """torch fp32 statement of the kernel's contract: s per row, the scaled
    gate and up rounded to the activation dtype, then SiLU(gate) * up."""
    dtype, inter = gu.dtype, gu.shape[-1] // 2
    s = torch.rsqrt(hidden.float().pow(2).mean(-1, keepdim=True) + eps)
    gate = (gu[..., :inter].float() * s).to(dtype).float()
    up = (gu[..., inter:].float() * s).to(dtype).float()
    return ((gate / (1 + torch.exp(-gate))).to(dtype).float() * up).to(dtype)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize(("rows", "dim", "inter"), [(1, 576, 1536), (5, 2048, 8192), (3, 64, 256), (2, 100, 12),
                                                   (4, 4096, 1024), (1, 8192, 64)])
def test_rms_silu_mul_matches_torch(dtype, rows, dim, inter):
    g = torch.Generator(device="cuda").manual_seed(rows * 31 + dim + inter)
    hidden = (4 * torch.randn(rows, dim, generator=g, device="cuda")).to(dtype)
    gu = (3 * torch.randn(rows, 2 * inter, generator=g, device="cuda")).to(dtype)
    out = torch.empty(rows, inter, dtype=dtype, device="cuda")
    ops.rms_silu_mul(gu, hidden, out, 1e-5)
    want = rms_silu_ref(gu, hidden, 1e-5)
    # s may differ from torch's in its last bit (another summation order)
    if dtype == torch.bfloat16:
        assert torch.allclose(out.float(), want.float(), rtol=2 ** -6, atol=1e-5)
        assert (out != want).float().mean().item() < 0.02
    else:
        assert torch.allclose(out, want, rtol=1e-5, atol=1e-6), (out - want).abs().max()


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_norm_after_projection_equals_norm_before(dtype):
    """The identity the forward relies on: projecting the unnormalised stream
    with the norm weight folded into W's columns, then this kernel, gives
    what RMSNorm -> projection -> SiLU*up gives, up to rounding.  A wrong
    fold (rows instead of columns, a missing weight) or a wrong scale is far
    outside the bound."""
    g = torch.Generator(device="cuda").manual_seed(5)
    rows, dim, inter = 5, 2048, 1024
    hidden = (4 * torch.randn(rows, dim, generator=g, device="cuda")).to(dtype)
    weight = (1 + 0.3 * torch.randn(dim, generator=g, device="cuda")).to(dtype)
    w = (0.02 * torch.randn(2 * inter, dim, generator=g, device="cuda")).to(dtype)
    x = torch.empty_like(hidden)
    ops.add_rmsnorm(hidden.clone(), None, weight, x, 1e-5)
    before = torch.empty(rows, inter, dtype=dtype, device="cuda")
    ops.silu_mul(torch.nn.functional.linear(x, w), before)
    folded = (w.float() * weight.float()).to(dtype)
    after = torch.empty_like(before)
    ops.rms_silu_mul(torch.nn.functional.linear(hidden, folded), hidden, after, 1e-5)
    tol = 3e-2 if dtype == torch.bfloat16 else 1e-4
    scale = before.float().abs().max().item()
    assert (after.float() - before.float()).abs().max().item() < tol * scale
    if dtype == torch.float32:
        assert torch.allclose(after, before, rtol=1e-4, atol=1e-6)


def test_rms_silu_rows_do_not_depend_on_the_call():
    """Each row's result is the same whether it comes with 5 rows or alone."""
    g = torch.Generator(device="cuda").manual_seed(9)
    hidden = torch.randn(5, 2048, generator=g, device="cuda").to(torch.bfloat16)
    gu = torch.randn(5, 16384, generator=g, device="cuda").to(torch.bfloat16)
    all_rows = ops.rms_silu_mul(gu, hidden, torch.empty(5, 8192, dtype=torch.bfloat16, device="cuda"), 1e-5)
    for r in range(5):
        one = ops.rms_silu_mul(gu[r:r + 1], hidden[r:r + 1], torch.empty(1, 8192, dtype=torch.bfloat16, device="cuda"),
                               1e-5)
        assert torch.equal(one, all_rows[r:r + 1])
