"""Output head kernels (specdec_head_logits, specdec_head_probabilities)
against fp64 products of the same bf16 operands and against torch's
softmax: the fp32 logits of lm/forward.py:71-84 and the probabilities of
lm/sampling.py:13-18.

The bf16 products are exact in fp32, so the logits differ from the fp64
ones only by the fp32 accumulation: bounded here by 1e-5 of the largest
|logit| (a dropped or repeated k-step is off by far more).  Probabilities
meet the reference's 1e-5 relative bound against the softmax of the fp64
logits.  Row invariance, the strided outputs, graph replays and the
statistics fallback are compared bit for bit.
"""
import pytest
import torch

from specdec import ops

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda", 0)


def operands(rows, hidden, vocab, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    x = (torch.randn(rows, hidden, generator=g) * scale).to(torch.bfloat16)
    w = (torch.randn(vocab, hidden, generator=g) * 0.02).to(torch.bfloat16)
    return x, w


def exact_logits(x, w):
    return x.double() @ w.double().t()


SHAPES = [(1, 2048, 49152), (5, 2048, 49152), (1, 576, 49152), (3, 576, 1000), (16, 64, 4099), (40, 2048, 3001),
          (70, 576, 2053)]


@pytest.mark.parametrize("rows,hidden,vocab", SHAPES)
def test_logits_match_fp64_products(rows, hidden, vocab):
    x, w = operands(rows, hidden, vocab, seed=rows + vocab)
    got = ops.head_logits(x.to(DEV), w.to(DEV)).cpu().double()
    want = exact_logits(x, w)
    assert got.shape == (rows, vocab)
    err = (got - want).abs().max().item()
    assert err <= 1e-5 * want.abs().max().item(), err


@pytest.mark.parametrize("rows,hidden,vocab", [(5, 2048, 49152), (16, 576, 4099), (40, 2048, 3001), (70, 64, 999)])
def test_row_logits_do_not_depend_on_the_other_rows(rows, hidden, vocab):
    x, w = operands(rows, hidden, vocab, seed=3)
    xd, wd = x.to(DEV), w.to(DEV)
    together = ops.head_logits(xd, wd)
    for r in range(rows):
        assert torch.equal(ops.head_logits(xd[r:r + 1], wd), together[r:r + 1]), r
    # every prefix of the rows too (column tiles of 16, 32 and 64 rows, and passes)
    for m in (1, 7, 17, 33, 65):
        if m <= rows:
            assert torch.equal(ops.head_logits(xd[:m], wd), together[:m]), m


@pytest.mark.parametrize("temperature", [1.0, 0.8, 0.3])
@pytest.mark.parametrize("rows,hidden,vocab", [(1, 2048, 49152), (5, 2048, 49152), (4, 576, 49152), (16, 576, 4099),
                                               (3, 64, 1000)])
def test_fused_probabilities_match_softmax(rows, hidden, vocab, temperature):
    x, w = operands(rows, hidden, vocab, seed=11, scale=2.0)
    xd, wd = x.to(DEV), w.to(DEV)
    lg = torch.empty(rows, vocab, device=DEV)
    p = ops.head_probabilities(xd, wd, temperature, logits_out=lg)
    # the logits it normalised are head_logits' bits
    assert torch.equal(lg, ops.head_logits(xd, wd))
    want = torch.softmax(exact_logits(x, w) / temperature, dim=-1)
    got = p.cpu().double()
    rel = ((got - want).abs() / want).max().item()
    # 1e-5 at the contract's temperatures; at T = 0.3 the fp32 logit and
    # exponent roundings are amplified 1/T-fold in the far tail (2e-5 seen)
    assert rel < (1e-5 if temperature >= 0.8 else 5e-5), rel
    # and the separate softmax kernel on the same logits agrees as closely
    sep = ops.probabilities(lg, temperature).cpu().double()
    assert ((got - sep).abs() / sep).max().item() < 1e-5


@pytest.mark.parametrize("rows,hidden,vocab", [(1, 2048, 49152), (5, 2048, 49152), (8, 576, 49152), (16, 64, 3001)])
def test_fused_argmax_is_the_lowest_id_among_ties(rows, hidden, vocab):
    x, w = operands(rows, hidden, vocab, seed=5)
    # plant exact ties: for each row, copies of one vocab row at a higher id
    # and at a lower id than the row's winner
    xd, wd = x.to(DEV), w.to(DEV)
    top = ops.head_logits(xd, wd).argmax(-1).cpu()
    w2 = w.clone()
    for r in range(rows):
        t = int(top[r])
        w2[(t + 1 + 97 * r) % vocab] = w[t]  # a tie somewhere else in the vocab
    wd2 = w2.to(DEV)
    lg = ops.head_logits(xd, wd2)
    want_idx = torch.tensor([int((lg[r] == lg[r].max()).nonzero()[0]) for r in range(rows)])
    idx = torch.full((rows,), -1, dtype=torch.int64, device=DEV)
    p = ops.head_probabilities(xd, wd2, 0.0, index_out=idx)
    assert torch.equal(idx.cpu(), want_idx)
    assert torch.equal(p.cpu(), torch.nn.functional.one_hot(want_idx, vocab).float())
    # the argmax of the logits torch sees agrees
    assert torch.equal(lg.argmax(-1).cpu(), want_idx)


@pytest.mark.parametrize("temperature", [0.0, 0.8])
def test_fused_rows_do_not_depend_on_the_other_rows(temperature):
    x, w = operands(5, 2048, 49152, seed=21, scale=2.0)
    xd, wd = x.to(DEV), w.to(DEV)
    together = ops.head_probabilities(xd, wd, temperature)
    for r in range(5):
        assert torch.equal(ops.head_probabilities(xd[r:r + 1], wd, temperature), together[r:r + 1]), r


@pytest.mark.parametrize("temperature", [0.0, 1.0, 0.8])
def test_statistics_fallback_has_the_same_bits(temperature):
    """spin = 0: no workgroup waits for the others; each computes every slice
    statistic it has not seen itself.  Same bits as the meeting."""
    x, w = operands(5, 576, 49152, seed=8, scale=2.0)
    xd, wd = x.to(DEV), w.to(DEV)
    idx_a = torch.zeros(5, dtype=torch.int64, device=DEV)
    idx_b = torch.zeros(5, dtype=torch.int64, device=DEV)
    kw = {"index_out": idx_a} if temperature == 0.0 else {}
    met = ops.head_probabilities(xd, wd, temperature, **kw)
    kw = {"index_out": idx_b} if temperature == 0.0 else {}
    alone = ops.head_probabilities(xd, wd, temperature, spin=0, **kw)
    assert torch.equal(met, alone)
    assert torch.equal(idx_a, idx_b)


def test_strided_outputs_and_calls_of_changing_shapes_share_the_workspace():
    """Writes into row-strided views ([B, steps, V] step slices, index
    columns), with calls of three vocabularies and row counts in turn
    through the one workspace: every call's statistics are its own."""
    cases = [(4, 576, 49152, 0.0), (3, 64, 1000, 0.7), (1, 2048, 49152, 1.0), (4, 576, 49152, 0.9),
             (16, 64, 1000, 0.0), (2, 2048, 49152, 0.0)]
    for i, (rows, hidden, vocab, t) in enumerate(cases):
        x, w = operands(rows, hidden, vocab, seed=40 + i, scale=2.0)
        xd, wd = x.to(DEV), w.to(DEV)
        q = torch.full((rows, 3, vocab), -1.0, device=DEV)
        toks = torch.full((rows, 3), -1, dtype=torch.int64, device=DEV)
        ops.head_probabilities(xd, wd, t, out=q[:, 1], index_out=toks[:, 1] if t == 0.0 else None)
        lg = ops.head_logits(xd, wd)
        if t == 0.0:
            want_idx = lg.argmax(-1)
            assert torch.equal(toks[:, 1], want_idx)
            assert torch.equal(q[:, 1], torch.nn.functional.one_hot(want_idx, vocab).float())
        else:
            want = ops.probabilities(lg, t)
            assert ((q[:, 1] - want).abs() / want).max().item() < 1e-5
        assert bool((q[:, 0] == -1).all()) and bool((q[:, 2] == -1).all())  # neighbours untouched
        assert bool((toks[:, 0] == -1).all()) and bool((toks[:, 2] == -1).all())


@pytest.mark.parametrize("temperature", [0.0, 0.8])
def test_graph_replays_match_eager_calls(temperature):
    """A captured fused call replayed on fresh inputs, eager work in between:
    each replay's output equals an eager call on the same inputs."""
    rows, hidden, vocab = 5, 2048, 49152
    _, w = operands(rows, hidden, vocab, seed=60)
    wd = w.to(DEV)
    xs = torch.zeros(rows, hidden, dtype=torch.bfloat16, device=DEV)
    ops.head_workspace(DEV)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        ops.head_probabilities(xs, wd, temperature)
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = ops.head_probabilities(xs, wd, temperature)
    for i in range(4):
        x, _ = operands(rows, hidden, 1, seed=70 + i, scale=2.0)
        xs.copy_(x.to(DEV))
        graph.replay()
        torch.cuda.synchronize()
        eager = ops.head_probabilities(xs, wd, temperature)
        ops.head_logits(xs, wd)  # other work between replays
        torch.cuda.synchronize()
        assert torch.equal(out, eager), i


def test_unsupported_shapes_are_refused():
    x, w = operands(17, 64, 1000, seed=1)
    with pytest.raises(ValueError):
        ops.head_probabilities(x.to(DEV), w.to(DEV), 1.0)
    x, w = operands(2, 48, 1000, seed=1)  # hidden not a multiple of 32
    with pytest.raises(NotImplementedError):
        ops.head_logits(x.to(DEV), w.to(DEV))
