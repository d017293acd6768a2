"""specdec_linear -- the bias-free projections of lm/forward.py:56-58,63-64
at decode sizes -- against fp64 products of the same bf16 operands.

The bf16 products are exact in fp32, so a result differs from the fp64 one
by the fp32 accumulation and the final rounding to bf16: at most half a
bf16 step of the exact value plus 1e-5 of sum |x_k w_k| (a dropped,
repeated or transposed k-step is off by far more).  Row invariance and the
residual add (`accumulate`, one rounding of the product plus the old
value) is held to the same bound; rows are compared bit for bit with the
kernel's own calls of other row counts."""
import pytest
import torch

from specdec import ops

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda", 0)


def operands(rows, k, n, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(rows, k, generator=g).to(torch.bfloat16)
    w = (torch.randn(n, k, generator=g) * 0.05).to(torch.bfloat16)
    return x, w


def half_step(v):
    """Half a bf16 step at |v| (8 significant bits)."""
    e = torch.floor(torch.log2(v.abs().clamp_min(1e-30)))
    return torch.pow(2.0, e - 8)


def check(got, x, w, base=None):
    exact = x.double() @ w.double().t()
    if base is not None:
        exact = exact + base.double()
    mag = x.double().abs() @ w.double().abs().t()
    err = (got.double() - exact).abs()
    bound = half_step(exact) + 1e-5 * mag
    assert bool((err <= bound).all()), (err - bound).max().item()


# draft (576 wide) and target (2048 / 8192 wide) projections, odd sizes,
# more than one 16-row tile
SHAPES = [(1, 576, 960), (1, 576, 3072), (1, 1536, 576), (5, 2048, 6144), (5, 8192, 2048), (3, 64, 100),
          (16, 96, 33), (17, 2048, 2048), (40, 576, 1000), (64, 8192, 48)]


@pytest.mark.parametrize("rows,k,n", SHAPES)
def test_linear_matches_fp64_products(rows, k, n):
    x, w = operands(rows, k, n, seed=rows * 7 + n)
    got = ops.linear(x.to(DEV), w.to(DEV)).cpu()
    assert got.shape == (rows, n) and got.dtype == torch.bfloat16
    check(got, x, w)


@pytest.mark.parametrize("rows,k,n", [(1, 576, 576), (5, 2048, 2048), (20, 1536, 576)])
def test_accumulate_adds_before_the_rounding(rows, k, n):
    x, w = operands(rows, k, n, seed=3)
    base = torch.randn(rows, n, generator=torch.Generator().manual_seed(4)).to(torch.bfloat16)
    out = base.to(DEV)
    ops.linear(x.to(DEV), w.to(DEV), out=out, accumulate=True)
    # one rounding of the exact sum plus the old value (two roundings, the
    # product's and the add's, would miss the bound near cancellations)
    check(out.cpu(), x, w, base)


@pytest.mark.parametrize("rows,k,n", [(5, 2048, 6144), (40, 576, 1000), (64, 8192, 48), (48, 64, 40),
                                      (16, 8192, 2048)])
def test_rows_do_not_depend_on_the_other_rows(rows, k, n):
    """Calls of 1 to 64 rows (one to four 16-row column tiles per wave; one
    wave for K = 64, up to eight otherwise): each row has the bits of the
    same row computed alone."""
    x, w = operands(rows, k, n, seed=5)
    xd, wd = x.to(DEV), w.to(DEV)
    together = ops.linear(xd, wd)
    for r in range(rows):
        assert torch.equal(ops.linear(xd[r:r + 1], wd), together[r:r + 1]), r
    for m in (1, 5, 8, 9, 16, 17, 33):
        if m <= rows:
            assert torch.equal(ops.linear(xd[:m], wd), together[:m]), m


def test_strided_rows_and_outputs():
    """x rows out of a wider tensor (row stride > K) and out a column block
    of a wider tensor: neighbours untouched."""
    rows, k, n = 6, 576, 960
    x, w = operands(rows, k, n, seed=9)
    wide = torch.zeros(rows, k + 64, dtype=torch.bfloat16, device=DEV)
    wide[:, 32:32 + k] = x.to(DEV)
    out = torch.full((rows, n + 48), 7.0, dtype=torch.bfloat16, device=DEV)
    ops.linear(wide[:, 32:32 + k], w.to(DEV), out=out[:, 16:16 + n])
    check(out[:, 16:16 + n].cpu(), x, w)
    assert bool((out[:, :16] == 7).all()) and bool((out[:, 16 + n:] == 7).all())


def test_graph_replays_match_eager_calls():
    rows, k, n = 5, 2048, 2048
    _, w = operands(rows, k, n, seed=11)
    wd = w.to(DEV)
    xs = torch.zeros(rows, k, dtype=torch.bfloat16, device=DEV)
    out = torch.zeros(rows, n, dtype=torch.bfloat16, device=DEV)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        ops.linear(xs, wd, out=out)
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        ops.linear(xs, wd, out=out)
    for i in range(3):
        x, _ = operands(rows, k, 1, seed=20 + i)
        xs.copy_(x.to(DEV))
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, ops.linear(xs, wd)), i


def test_unsupported_shapes_are_refused():
    x, w = operands(65, 64, 16, seed=1)
    with pytest.raises(NotImplementedError):
        ops.linear(x.to(DEV), w.to(DEV))
    x, w = operands(2, 48, 16, seed=1)  # K not a multiple of 32
    with pytest.raises(NotImplementedError):
        ops.linear(x.to(DEV), w.to(DEV))


@pytest.mark.parametrize("rows,k,inter,hdim,same", [(1, 576, 1536, 576, True), (5, 2048, 8192, 2048, True),
                                                     (16, 576, 1536, 576, True), (3, 64, 104, 64, False),
                                                     (40, 576, 1536, 576, True), (7, 96, 48, 1024, False)])
def test_linear_silu_equals_linear_then_rms_silu_mul(rows, k, inter, hdim, same):
    """The gate/up projection with the MLP's norm scale and SiLU·up in its
    epilogue has the bits of specdec_linear followed by rms_silu_mul (the
    decode-sized MLP of lm/forward.py: x is the residual row itself), also
    for a gate half that ends inside a 16-feature tile."""
    g = torch.Generator().manual_seed(rows * 13 + inter)
    w = (torch.randn(2 * inter, k, generator=g) * 0.05).to(torch.bfloat16).to(DEV)
    hidden = (torch.randn(rows, hdim, generator=g) * 3).to(torch.bfloat16).to(DEV)
    x = hidden if same else (torch.randn(rows, k, generator=g)).to(torch.bfloat16).to(DEV)
    eps = 1e-5
    fused = torch.full((rows, inter), 7.0, dtype=torch.bfloat16, device=DEV)
    ops.linear_silu(x, w, hidden, fused, eps)
    two = torch.empty(rows, inter, dtype=torch.bfloat16, device=DEV)
    ops.rms_silu_mul(ops.linear(x, w), hidden, two, eps)
    assert torch.equal(fused, two)
    # and the activation is what transformers computes from the same bf16 gate/up values
    gu = ops.linear(x, w).float().cpu()
    s = torch.rsqrt(hidden.float().cpu().pow(2).mean(-1, keepdim=True) + eps)
    gate = (s * gu[:, :inter]).to(torch.bfloat16).float()
    up = (s * gu[:, inter:]).to(torch.bfloat16).float()
    want = (torch.nn.functional.silu(gate).to(torch.bfloat16).float() * up).to(torch.bfloat16)
    assert (fused.cpu().float() - want.float()).abs().max().item() <= 2 ** -6 * want.float().abs().max().item()


@pytest.mark.parametrize("rows,k,n", [(1, 576, 960), (1, 1536, 576), (5, 2048, 6144), (5, 8192, 2048), (16, 96, 48),
                                      (40, 576, 1008), (64, 8192, 48)])
def test_tiled_weight_gives_the_same_bits(rows, k, n):
    """The weight in its tiled layout (each 16 x 32 block 1 KB contiguous in
    the lanes' order) is the same arithmetic as the row-major weight: plain
    and accumulating projections are equal bit for bit, at every row count
    and instance."""
    x, w = operands(rows, k, n, seed=rows + k + n)
    xd, wd = x.to(DEV), w.to(DEV)
    wt = ops.tile_weight(wd)
    assert torch.equal(ops.linear(xd, wt), ops.linear(xd, wd))
    base = (torch.randn(rows, n, generator=torch.Generator().manual_seed(n)) * 2).to(torch.bfloat16).to(DEV)
    a, b = base.clone(), base.clone()
    ops.linear(xd, wd, out=a, accumulate=True)
    ops.linear(xd, wt, out=b, accumulate=True)
    assert torch.equal(a, b)


@pytest.mark.parametrize("rows,k,inter", [(1, 576, 1536), (5, 2048, 8192), (40, 576, 1536)])
def test_linear_silu_tiled_weight_gives_the_same_bits(rows, k, inter):
    g = torch.Generator().manual_seed(rows + inter)
    w = (torch.randn(2 * inter, k, generator=g) * 0.05).to(torch.bfloat16).to(DEV)
    hidden = (torch.randn(rows, k, generator=g) * 3).to(torch.bfloat16).to(DEV)
    a = torch.empty(rows, inter, dtype=torch.bfloat16, device=DEV)
    b = torch.empty_like(a)
    ops.linear_silu(hidden, w, hidden, a, 1e-5)
    ops.linear_silu(hidden, ops.tile_weight(w), hidden, b, 1e-5)
    assert torch.equal(a, b)
