"""Paged verify attention kernel vs SDPA on the gathered cache (the
reference's attention step), plus the cache write/gather and rollback."""
import random

import pytest
import torch

import oracle.forward as of
from cache.kv import KVCache
from specdec import ops

pytestmark = pytest.mark.gpu


def make_cache(layers, hkv, d, num_blocks, bs, dtype, seed):
    """A cache whose blocks are handed out in a seeded random order: a
    permutation of the pool is allocated and freed once so the LIFO stack
    yields shuffled block ids."""
    cache = KVCache(layers, hkv, d, num_blocks, bs, dtype, "cuda")
    perm = torch.randperm(num_blocks, generator=torch.Generator().manual_seed(seed)).tolist()
    cache.add(-1)
    cache.append([-1], [num_blocks * bs])
    # free in permuted order by rewriting the table before releasing it
    table = cache.tables[-1]
    cache.table_tensor[table.row, :num_blocks] = torch.tensor(perm, dtype=torch.int32, device="cuda")
    cache.free(-1)
    cache.flush()
    return cache


def padded(rows: list[torch.Tensor], width: int) -> torch.Tensor:
    """Per-row [Hkv, n_b, d] host tensors -> [B, Hkv, width, d] fp32, zeros past n_b."""
    hkv, d = rows[0].shape[0], rows[0].shape[2]
    out = torch.zeros(len(rows), hkv, width, d)
    for b, r in enumerate(rows):
        out[b, :, : r.shape[1]] = r.float()
    return out


def run_case(batch, lengths, h, hkv, bs, dtype, t_new, seed, rollback=True):
    """Two verify rounds over a shuffled pool, each followed by a rollback of
    a seeded number of rejected positions.  The expected output is SDPA over
    the K/V the test wrote, kept on the host (appends concatenated, rollbacks
    cut), never read back from the device; the device copy (cache.gather)
    must equal that host copy bit for bit."""
    d = 64
    g = torch.Generator().manual_seed(seed)
    nb = sum((L + 2 * t_new + 2 * bs) // bs + 1 for L in lengths) + 8
    cache = make_cache(1, hkv, d, nb, bs, dtype, seed)
    ids = list(range(batch))
    for s in ids:
        cache.add(s)
    # history: prefill each row to its length with random K/V
    step = cache.append(ids, lengths)
    kh = torch.randn(batch, hkv, max(lengths), d, generator=g).to(dtype)
    vh = torch.randn(batch, hkv, max(lengths), d, generator=g).to(dtype)
    cache.write(0, step, kh.cuda(), vh.cuda())
    host_k = [kh[b, :, : lengths[b]] for b in range(batch)]
    host_v = [vh[b, :, : lengths[b]] for b in range(batch)]
    outs = []
    for rnd in range(2):
        step = cache.append(ids, [t_new] * batch)
        q = torch.randn(batch, t_new, h, d, generator=g).to(dtype)
        kn = torch.randn(batch, hkv, t_new, d, generator=g).to(dtype)
        vn = torch.randn(batch, hkv, t_new, d, generator=g).to(dtype)
        cache.write(0, step, kn.cuda(), vn.cuda())
        host_k = [torch.cat([host_k[b], kn[b]], dim=1) for b in range(batch)]
        host_v = [torch.cat([host_v[b], vn[b]], dim=1) for b in range(batch)]
        out = torch.zeros(batch, t_new, h * d, dtype=dtype, device="cuda")
        qd = q.reshape(batch, t_new, h * d).cuda()
        ops.paged_attention(qd, qd.stride(1), cache.k[0], cache.v[0], cache.table_tensor, step.meta, batch,
                            t_new, h, hkv, d, bs, d ** -0.5, step.max_total, out, out.stride(1))
        k_all, v_all = padded(host_k, step.max_total), padded(host_v, step.max_total)
        dev_k, dev_v = cache.gather(0, step)
        assert torch.equal(dev_k.cpu().float(), k_all) and torch.equal(dev_v.cpu().float(), v_all)
        want = of.attention(q.transpose(1, 2).float(), k_all, v_all, torch.tensor(step.past), torch.tensor(step.total),
                            d ** -0.5)
        got = out.view(batch, t_new, h, d).transpose(1, 2).float().cpu()
        outs.append((got, want))
        if rollback:
            rng = random.Random(seed * 7 + rnd)
            for b, s in enumerate(ids):
                keep = step.past[b] + 1 + rng.randint(0, t_new - 1)
                cache.truncate(s, keep)
                host_k[b], host_v[b] = host_k[b][:, :keep], host_v[b][:, :keep]
    return outs


@pytest.mark.parametrize("length", [512, 1024, 2048, 4096])
@pytest.mark.parametrize("batch", [1, 4, 8])
def test_config2_bf16_matches_sdpa(batch, length):
    """32/32 heads, d=64, bs=16, bf16, k+1=5 queries, shuffled pool, rollback."""
    lengths = [length - 3 * b for b in range(batch)]
    for got, want in run_case(batch, lengths, 32, 32, 16, torch.bfloat16, 5, seed=batch * 10000 + length):
        err = (got - want).abs().max().item()
        assert err < 2e-2, err


@pytest.mark.parametrize("bs", [1, 3, 4, 16, 32])
@pytest.mark.parametrize("heads", [(4, 2), (9, 3), (8, 8)])
def test_fp32_any_block_size_and_gqa(bs, heads):
    h, hkv = heads
    for got, want in run_case(3, [37, 5, 70], h, hkv, bs, torch.float32, 5, seed=bs * 100 + h):
        assert torch.allclose(got, want, atol=2e-5, rtol=1e-5), (got - want).abs().max()


@pytest.mark.parametrize("bs", [4, 16])
def test_bf16_gqa_small_blocks(bs):
    for got, want in run_case(2, [300, 45], 9, 3, bs, torch.bfloat16, 1, seed=bs):
        assert (got - want).abs().max().item() < 2e-2


@pytest.mark.parametrize("L", [300, 509, 1000, 2044, 4090])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_verify_rows_equal_decode_rows_bitwise(dtype, L):
    """The same query at the same position gives identical bits whether it is
    verified among k+1 tokens or decoded alone: the reduction order depends
    only on key positions (the property the greedy identity relies on).  At
    L = 2044 the verify call needs 5 splits of 512 (split kernel + combine
    kernel) while the first decode calls need 4 (one 16-wave workgroup
    folding them in LDS): both paths must give the same bits."""
    d, h, hkv, bs = 64, 32, 32, 16
    g = torch.Generator().manual_seed(5)
    cache = make_cache(1, hkv, d, (L + 5) // bs + 8, bs, dtype, 1)
    cache.add(0)
    step = cache.append([0], [L + 5])
    kh = torch.randn(1, hkv, L + 5, d, generator=g).to(dtype).cuda()
    vh = torch.randn(1, hkv, L + 5, d, generator=g).to(dtype).cuda()
    cache.write(0, step, kh, vh)
    q = torch.randn(1, 5, h * d, generator=g).to(dtype).cuda()
    cache.truncate(0, L)
    step5 = cache.append([0], [5])
    out5 = torch.zeros(1, 5, h * d, dtype=dtype, device="cuda")
    ops.paged_attention(q, q.stride(1), cache.k[0], cache.v[0], cache.table_tensor, step5.meta, 1, 5, h, hkv, d,
                        bs, 0.125, step5.max_total, out5, out5.stride(1))
    for t in range(5):
        cache.truncate(0, L + t)
        step1 = cache.append([0], [1])
        out1 = torch.zeros(1, 1, h * d, dtype=dtype, device="cuda")
        q1 = q[:, t:t + 1].contiguous()
        ops.paged_attention(q1, q1.stride(1), cache.k[0], cache.v[0], cache.table_tensor, step1.meta, 1, 1, h, hkv,
                            d, bs, 0.125, step1.max_total, out1, out1.stride(1))
        assert torch.equal(out1[0, 0], out5[0, t]), t


@pytest.mark.parametrize("L", [4090, 4100])
def test_batch8_verify_rows_equal_batch1_decode_rows_bitwise(L):
    """Batch 8 against one row decoded alone at batch 1, both with split
    partials folded by the combine kernel (L = 4100: eight full splits and
    a short ninth).  The fold tree depends only on key positions, so the
    bits are the same."""
    d, h, hkv, bs, B = 64, 32, 32, 16, 8
    g = torch.Generator().manual_seed(21)
    cache = make_cache(1, hkv, d, B * ((L + 8) // bs + 2) + 8, bs, torch.bfloat16, 6)
    ids = list(range(B))
    for s in ids:
        cache.add(s)
    lengths = [L - 7 * b for b in range(B)]
    step = cache.append(ids, [n + 5 for n in lengths])
    cache.write(0, step, torch.randn(B, hkv, L + 5, d, generator=g).to(torch.bfloat16).cuda(),
                torch.randn(B, hkv, L + 5, d, generator=g).to(torch.bfloat16).cuda())
    q = torch.randn(B, 5, h * d, generator=g).to(torch.bfloat16).cuda()
    for s, n in zip(ids, lengths):
        cache.truncate(s, n)
    step8 = cache.append(ids, [5] * B)
    out8 = torch.zeros(B, 5, h * d, dtype=torch.bfloat16, device="cuda")
    ops.paged_attention(q, q.stride(1), cache.k[0], cache.v[0], cache.table_tensor, step8.meta, B, 5, h, hkv, d, bs,
                        0.125, step8.max_total, out8, out8.stride(1))
    for row in (0, 5):
        for t in range(5):
            cache.truncate(row, lengths[row] + t)
            step1 = cache.append([row], [1])
            out1 = torch.zeros(1, 1, h * d, dtype=torch.bfloat16, device="cuda")
            q1 = q[row:row + 1, t:t + 1].contiguous()
            ops.paged_attention(q1, q1.stride(1), cache.k[0], cache.v[0], cache.table_tensor, step1.meta, 1, 1, h,
                                hkv, d, bs, 0.125, step1.max_total, out1, out1.stride(1))
            assert torch.equal(out1[0, 0], out8[row, t]), (row, t)


def test_prefill_many_query_tiles():
    """A 200-token prefill (13 query tiles per head) against SDPA."""
    for got, want in run_case(2, [0, 17], 4, 2, 16, torch.float32, 200, seed=3, rollback=False):
        assert torch.allclose(got, want, atol=2e-5, rtol=1e-5)


def test_repeated_split_combines_stay_exact():
    """Many back-to-back launches over the same workspace (every call splits
    9 ways and combines in a second kernel): each result is compared with
    SDPA over the host K/V, so a stale or overwritten partial shows."""
    h = 32
    cache, step, _, host = _filled(1, [4096], seed=11)
    g = torch.Generator().manual_seed(11)
    outs, qs = [], []
    for i in range(40):
        qd = torch.randn(1, 5, h * 64, generator=g).to(torch.bfloat16).cuda()
        outs.append(_attend(cache, step, qd, None))
        qs.append(qd)
    for qd, out in zip(qs, outs):
        assert (_got(out) - _want(qd, step, host)).abs().max().item() < 2e-2


@pytest.mark.parametrize("split", [256, 512, 2048, -1])
@pytest.mark.parametrize("heads", [(32, 32), (9, 3)])
def test_explicit_split_sizes(split, heads):
    """Caller-chosen splits against SDPA; -1 is the draft's flat policy (one
    16-wave workgroup striding every key)."""
    h, hkv = heads
    cache, step, q, host = _filled(2, [1500, 333], seed=split + h, h=h, hkv=hkv, t_new=1)
    out = torch.zeros(2, 1, h * 64, dtype=torch.bfloat16, device="cuda")
    ops.paged_attention(q, q.stride(1), cache.k[0], cache.v[0], cache.table_tensor, step.meta, 2, 1, h, hkv, 64, 16,
                        0.125, step.max_total, out, out.stride(1), ops.AttentionWorkspace(q.device), split)
    assert (_got(out, h) - _want(q, step, host, h)).abs().max().item() < 2e-2


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize(("bs", "t_new", "lengths"), [(16, 5, [1000, 37]), (4, 3, [50, 9]), (16, 200, [0, 300])])
def test_fused_rope_append_equals_separate_kernels(dtype, bs, t_new, lengths):
    """rope_paged_attention == rope_append followed by paged_attention: the
    attention output and the pool contents at the new positions, bit for bit."""
    from lm.model import LlamaShape, rope_tables

    h, hkv, d = 8, 4, 64
    shape = LlamaShape(vocab_size=8, hidden_size=h * d, num_hidden_layers=1, num_attention_heads=h,
                       num_key_value_heads=hkv, intermediate_size=8, rope_theta=10000.0)
    cos, sin = (x.cuda() for x in rope_tables(shape, 2048))
    g = torch.Generator().manual_seed(bs * 31 + t_new)
    caches = [make_cache(1, hkv, d, 200, bs, dtype, 3) for _ in range(2)]
    hist = [torch.randn(2, hkv, max(max(lengths), 1), d, generator=g).to(dtype).cuda() for _ in range(2)]
    qkv = torch.randn(2, t_new, (h + 2 * hkv) * d, generator=g).to(dtype).cuda()
    outs = []
    for which, cache in enumerate(caches):
        for s in (0, 1):
            cache.add(s)
        step = cache.append([0, 1], lengths)
        if max(lengths) > 0:
            cache.write(0, step, hist[0], hist[1])
        step = cache.append([0, 1], [t_new, t_new])
        out = torch.zeros(2, t_new, h * d, dtype=dtype, device="cuda")
        x = qkv.clone()
        if which == 0:
            ops.rope_append(x, h, hkv, d, cos, sin, step.meta, 2, t_new, cache.table_tensor, bs, cache.k[0],
                            cache.v[0])
            ops.paged_attention(x, x.stride(1), cache.k[0], cache.v[0], cache.table_tensor, step.meta, 2, t_new, h,
                                hkv, d, bs, 0.125, step.max_total, out, out.stride(1))
        else:
            ops.rope_paged_attention(x, cos, sin, cache.k[0], cache.v[0], cache.table_tensor, step.meta, 2, t_new, h,
                                     hkv, d, bs, 0.125, step.max_total, out, out.stride(1))
        k_all, v_all = cache.gather(0, step)
        outs.append((out, k_all, v_all))
    for a, b in zip(outs[0], outs[1]):
        assert torch.equal(a, b)


def _filled(batch, lengths, seed, h=32, hkv=32, t_new=5):
    """A bf16 cache of `batch` rows with lengths[b] cached keys each (random
    K/V, shuffled blocks, block 16), t_new more appended, and q for them.
    The K/V written are kept on the host: returns (cache, step, q, host)
    with host = (K, V) [B, Hkv, max_total, d] fp32, zeros past each row."""
    d, bs = 64, 16
    g = torch.Generator().manual_seed(seed)
    cache = make_cache(1, hkv, d, sum((n + t_new) // bs + 2 for n in lengths) + 8, bs, torch.bfloat16, seed)
    ids = list(range(batch))
    for s in ids:
        cache.add(s)
    step = cache.append(ids, list(lengths))
    kh = torch.randn(batch, hkv, max(lengths), d, generator=g).to(torch.bfloat16)
    vh = torch.randn(batch, hkv, max(lengths), d, generator=g).to(torch.bfloat16)
    cache.write(0, step, kh.cuda(), vh.cuda())
    step = cache.append(ids, [t_new] * batch)
    kn = torch.randn(batch, hkv, t_new, d, generator=g).to(torch.bfloat16)
    vn = torch.randn(batch, hkv, t_new, d, generator=g).to(torch.bfloat16)
    cache.write(0, step, kn.cuda(), vn.cuda())
    q = torch.randn(batch, t_new, h * d, generator=g).to(torch.bfloat16).cuda()
    host = tuple(padded([torch.cat([x[b, :, :n], y[b]], dim=1) for b, n in enumerate(lengths)], step.max_total)
                 for x, y in ((kh, kn), (vh, vn)))
    return cache, step, q, host


def _want(q, step, host, h=32):
    """SDPA over the host K/V for q [B, T, h*64] (the reference's attention step)."""
    b, t_new = q.shape[0], q.shape[1]
    return of.attention(q.view(b, t_new, h, 64).transpose(1, 2).float().cpu(), host[0], host[1],
                        torch.tensor(step.past), torch.tensor(step.total), 0.125)


def _got(out, h=32):
    b, t_new = out.shape[0], out.shape[1]
    return out.view(b, t_new, h, 64).transpose(1, 2).float().cpu()


def _attend(cache, step, q, ws, out=None, h=32, hkv=32):
    batch, t_new = q.shape[0], q.shape[1]
    ws = ws if ws is not None else ops.workspace_for(q.device)
    if out is None:
        out = torch.zeros(batch, t_new, h * 64, dtype=torch.bfloat16, device="cuda")
    ops.paged_attention(q, q.stride(1), cache.k[0], cache.v[0], cache.table_tensor, step.meta, batch, t_new, h, hkv,
                        64, cache.block_size, 0.125, step.max_total, out, out.stride(1), ws)
    return out


# (batch, cached lengths): 9 splits of 512 at batch 8, 6, ragged 2..9, 18
# (five groups of four in the combine) and 34 (two rounds of its
# eight-group fold); at batch 1 with 6, 9 and 14 splits the grid is small
# enough for the two-waves-per-SIMD split kernel
_SPLIT_SHAPES = [(8, [4100 - 7 * b for b in range(8)]), (1, [3000]), (3, [2600, 700, 4500]), (2, [9000, 5000]),
                 (1, [17000]), (1, [4100]), (1, [7000])]


def test_split_workspace_shared_across_shapes():
    """One workspace for calls of different shapes: the tile and split
    counts differ, so one call's partials lie where another's were.  Each
    result equals the same call on a fresh workspace bit for bit and
    matches SDPA."""
    built = [_filled(b, lengths, seed=40 + i) for i, (b, lengths) in enumerate(_SPLIT_SHAPES)]
    shared = ops.AttentionWorkspace(torch.device("cuda"))
    for rep in range(2):
        for i, (cache, step, q, host) in enumerate(built):
            got = _attend(cache, step, q, shared)
            fresh = _attend(cache, step, q, ops.AttentionWorkspace(torch.device("cuda")))
            torch.cuda.synchronize()
            assert torch.equal(got, fresh), (rep, i)
            if rep == 0:
                err = (_got(got) - _want(q, step, host)).abs().max().item()
                assert err < 2e-2, (i, err)


@pytest.mark.parametrize("shape", ["split", "split_b1", "tiled"])
def test_split_graph_replays_match_eager(shape):
    """A split-path call (split kernel + combine, at batch 2 or, with the
    two-waves-per-SIMD split kernel, at batch 1; or, at batch 8, one tiled
    launch) captured in a HIP graph: each replay -- with eager calls of
    another shape on the same workspace in between -- gives the eager
    bits."""
    from lm.graphs import _capture

    if shape == "split":
        cache, step, q, _ = _filled(2, [5000, 2600], seed=61)
    elif shape == "split_b1":
        cache, step, q, _ = _filled(1, [4100], seed=64)
    else:
        cache, step, q, _ = _filled(8, [3000 + 100 * b for b in range(8)], seed=63)
    other = _filled(3, [2600, 700, 4500], seed=62)[:3]
    ws = ops.AttentionWorkspace(torch.device("cuda"))
    ws.reserve(1 << 24)  # no growth inside the capture
    want = _attend(cache, step, q, ws)
    want_other = _attend(*other, ws)
    out = torch.zeros_like(want)
    graph, _ = _capture(lambda: _attend(cache, step, q, ws, out))
    for i in range(3):
        out.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, want), i
        assert torch.equal(_attend(*other, ws), want_other), i


def test_ragged_batch8_rows_equal_rows_verified_alone_bitwise():
    """Batch 8 with rows of 1 to 16 splits: the call runs one workgroup per
    split plus the combine kernel for every tile.  Each row verified alone
    at batch 1 takes the 16-wave path (up to four splits, folded in LDS) or
    the same split path; either way the bits are the same, and the batch
    result matches SDPA."""
    lengths = [7900, 100, 2500, 4100, 600, 7000, 3000, 1500]
    cache, step, q, host = _filled(8, lengths, seed=71)
    out8 = _attend(cache, step, q, ops.AttentionWorkspace(torch.device("cuda")))
    err = (_got(out8) - _want(q, step, host)).abs().max().item()
    assert err < 2e-2, err
    for row, n in enumerate(lengths):
        cache.truncate(row, n)
        step1 = cache.append([row], [5])
        q1 = q[row:row + 1].contiguous()
        out1 = _attend(cache, step1, q1, ops.AttentionWorkspace(torch.device("cuda")))
        assert torch.equal(out1[0], out8[row]), row


def test_tiled_batch8_rows_equal_rows_verified_alone_bitwise():
    """Batch 8 with rows of 1 to 12 splits (at most 6144 keys, 5 queries):
    256 tiles, one per CU, so the call runs tiled -- one 16-wave workgroup
    per tile whose wave groups take its splits in rounds, each wave keeping
    its per-split softmax state in LDS, folded at the end with the split
    kernel's and the combine's arithmetic.  Each row verified alone at
    batch 1 (16-wave or split + combine path) gives the same bits, and the
    batch result matches SDPA."""
    lengths = [6100, 100, 2500, 4100, 600, 5000, 3000, 1500]
    cache, step, q, host = _filled(8, lengths, seed=81)
    out8 = _attend(cache, step, q, ops.AttentionWorkspace(torch.device("cuda")))
    err = (_got(out8) - _want(q, step, host)).abs().max().item()
    assert err < 2e-2, err
    for row, n in enumerate(lengths):
        cache.truncate(row, n)
        step1 = cache.append([row], [5])
        q1 = q[row:row + 1].contiguous()
        out1 = _attend(cache, step1, q1, ops.AttentionWorkspace(torch.device("cuda")))
        assert torch.equal(out1[0], out8[row]), row


@pytest.mark.parametrize("bs", [16, 32])
def test_tiled_fused_rope_append_equals_separate_kernels(bs):
    """The tiled path (batch 8, 32 kv heads: a tile per CU; 7 to 8 splits)
    with the fused RoPE + append -- the appended tokens staged in LDS, the
    rest read from the pools -- gives the bits of rope_append followed by
    paged_attention, and leaves the same pool contents."""
    from lm.model import LlamaShape, rope_tables

    h = hkv = 32
    d, batch, t_new = 64, 8, 5
    shape = LlamaShape(vocab_size=8, hidden_size=h * d, num_hidden_layers=1, num_attention_heads=h,
                       num_key_value_heads=hkv, intermediate_size=8, rope_theta=10000.0)
    cos, sin = (x.cuda() for x in rope_tables(shape, 8192))
    g = torch.Generator().manual_seed(bs)
    lengths = [4000 - 300 * b for b in range(batch)]
    blocks = sum((n + t_new) // bs + 2 for n in lengths) + 8
    caches = [make_cache(1, hkv, d, blocks, bs, torch.bfloat16, 3) for _ in range(2)]
    hist = [torch.randn(batch, hkv, max(lengths), d, generator=g).to(torch.bfloat16).cuda() for _ in range(2)]
    qkv = torch.randn(batch, t_new, (h + 2 * hkv) * d, generator=g).to(torch.bfloat16).cuda()
    ids = list(range(batch))
    outs = []
    for which, cache in enumerate(caches):
        for s in ids:
            cache.add(s)
        step = cache.append(ids, lengths)
        cache.write(0, step, hist[0], hist[1])
        step = cache.append(ids, [t_new] * batch)
        out = torch.zeros(batch, t_new, h * d, dtype=torch.bfloat16, device="cuda")
        x = qkv.clone()
        if which == 0:
            ops.rope_append(x, h, hkv, d, cos, sin, step.meta, batch, t_new, cache.table_tensor, bs, cache.k[0],
                            cache.v[0])
            ops.paged_attention(x, x.stride(1), cache.k[0], cache.v[0], cache.table_tensor, step.meta, batch, t_new,
                                h, hkv, d, bs, 0.125, step.max_total, out, out.stride(1))
        else:
            ops.rope_paged_attention(x, cos, sin, cache.k[0], cache.v[0], cache.table_tensor, step.meta, batch,
                                     t_new, h, hkv, d, bs, 0.125, step.max_total, out, out.stride(1))
        k_all, v_all = cache.gather(0, step)
        outs.append((out, k_all, v_all))
    for x, y in zip(outs[0], outs[1]):
        assert torch.equal(x, y)


def _norm_case(batch, lengths, h, hkv, hidden_dim, split_tokens, t_new=5, seed=0):
    """Two identical caches; rope_paged_attention on q/k/v pre-scaled by each
    token's RMS factor vs on the raw projection with norm_of = the residual
    rows.  Each token's residual row is +-2^e_t (random signs, e_t in
    -2..2), so its mean square is exactly 4^e_t and the factor (eps = 0) is
    exactly 2^-e_t in any summation order: the two calls must agree bit for
    bit, and a scale applied to the wrong token, or missing from q, k or v,
    cannot."""
    from lm.model import LlamaShape, rope_tables

    d, bs = 64, 16
    shape = LlamaShape(vocab_size=8, hidden_size=h * d, num_hidden_layers=1, num_attention_heads=h,
                       num_key_value_heads=hkv, intermediate_size=8, rope_theta=10000.0)
    cos, sin = (x.cuda() for x in rope_tables(shape, max(lengths) + 64))
    g = torch.Generator().manual_seed(seed)
    expo = torch.randint(-2, 3, (batch, t_new, 1), generator=g).float()
    signs = torch.randint(0, 2, (batch, t_new, hidden_dim), generator=g).float() * 2 - 1
    hidden = (signs * torch.exp2(expo)).to(torch.bfloat16).cuda()
    factor = torch.exp2(-expo).to(torch.bfloat16).cuda()
    qkv = torch.randn(batch, t_new, (h + 2 * hkv) * d, generator=g).to(torch.bfloat16).cuda()
    blocks = sum((n + t_new) // bs + 2 for n in lengths) + 8
    hist = [torch.randn(batch, hkv, max(lengths), d, generator=g).to(torch.bfloat16).cuda() for _ in range(2)]
    ids = list(range(batch))
    outs = []
    for which in range(2):
        cache = make_cache(1, hkv, d, blocks, bs, torch.bfloat16, 3)
        for s in ids:
            cache.add(s)
        step = cache.append(ids, lengths)
        cache.write(0, step, hist[0], hist[1])
        step = cache.append(ids, [t_new] * batch)
        out = torch.zeros(batch, t_new, h * d, dtype=torch.bfloat16, device="cuda")
        x = qkv * factor if which == 0 else qkv.clone()
        ops.rope_paged_attention(x, cos, sin, cache.k[0], cache.v[0], cache.table_tensor, step.meta, batch, t_new, h,
                                 hkv, d, bs, 0.125, step.max_total, out, out.stride(1), split_tokens=split_tokens,
                                 norm_of=None if which == 0 else hidden, eps=0.0)
        k_all, v_all = cache.gather(0, step)
        outs.append((out, k_all, v_all))
    return outs


@pytest.mark.parametrize(("batch", "lengths", "heads", "hidden_dim", "split"), [
    (2, [300, 37], (32, 32), 2048, 0),  # one 16-wave workgroup per tile, grouped splits
    (2, [300, 37], (9, 3), 576, -1),  # the draft's flat split
    (1, [3000], (32, 32), 2048, 0),  # few 4-wave split workgroups, loads paired
    (3, [2600, 700, 4500], (32, 32), 2048, 0),  # 4-wave splits + combine
    (8, [4000 - 300 * b for b in range(8)], (32, 32), 2048, 0),  # tiled
])
def test_input_norm_in_attention_equals_prescaled_qkv(batch, lengths, heads, hidden_dim, split):
    ref, got = _norm_case(batch, lengths, heads[0], heads[1], hidden_dim, split)
    for a, b in zip(ref, got):
        assert torch.equal(a, b)


@pytest.mark.parametrize("lengths", [[300, 37], [1500, 700], [2000, 1]])
@pytest.mark.parametrize("heads,hidden_dim", [((9, 3), 576), ((32, 32), 2048), ((8, 1), 512)])
def test_latency_decode_step_input_norm_equals_prescaled_qkv(lengths, heads, hidden_dim):
    """A draft-style decode step (one new token per row, split -1: the 4-wave
    decode kernel, whose waves each compute the norm scale and take the new
    token's K and V from registers) with the norm finished inside equals the
    same step on pre-scaled q/k/v, output and pool contents bit for bit."""
    ref, got = _norm_case(len(lengths), lengths, heads[0], heads[1], hidden_dim, -1, t_new=1, seed=len(lengths) + heads[0])
    for a, b in zip(ref, got):
        assert torch.equal(a, b)


@pytest.mark.parametrize("bs", [16, 32])
@pytest.mark.parametrize("lengths", [[300, 37, 1], [1500, 2040]])
@pytest.mark.parametrize("heads", [(9, 3), (32, 32)])
def test_latency_decode_step_matches_oracle(bs, lengths, heads):
    """The decode kernel against the reference's decode step on the host
    (lm/forward.py:40-49, 53, 60-63 with one new token): RoPE of q and k at
    the row's position, the new K/V appended, SDPA over every cached key.
    The pool holds the host's rotated k and v bit for bit."""
    from lm.model import LlamaShape, rope_tables

    h, hkv = heads
    d, batch = 64, len(lengths)
    shape = LlamaShape(vocab_size=8, hidden_size=h * d, num_hidden_layers=1, num_attention_heads=h,
                       num_key_value_heads=hkv, intermediate_size=8, rope_theta=100000.0)
    cos_h, sin_h = rope_tables(shape, 2112)
    cos, sin = cos_h.cuda(), sin_h.cuda()
    g = torch.Generator().manual_seed(bs + h + lengths[0])
    cache = make_cache(1, hkv, d, sum(n // bs + 3 for n in lengths) + 8, bs, torch.bfloat16, 11)
    ids = list(range(batch))
    for s_ in ids:
        cache.add(s_)
    hist_k = [torch.randn(hkv, n, d, generator=g).to(torch.bfloat16) for n in lengths]
    hist_v = [torch.randn(hkv, n, d, generator=g).to(torch.bfloat16) for n in lengths]
    step = cache.append(ids, lengths)
    cache.write(0, step, padded(hist_k, max(lengths)).to(torch.bfloat16).cuda(),
                padded(hist_v, max(lengths)).to(torch.bfloat16).cuda())
    step = cache.append(ids, [1] * batch)
    qkv = torch.randn(batch, 1, (h + 2 * hkv) * d, generator=g).to(torch.bfloat16)
    out = torch.zeros(batch, 1, h * d, dtype=torch.bfloat16, device="cuda")
    ops.rope_paged_attention(qkv.cuda(), cos, sin, cache.k[0], cache.v[0], cache.table_tensor, step.meta, batch, 1, h,
                             hkv, d, bs, 0.125, step.max_total, out, out.stride(1), split_tokens=-1)
    q_all = qkv[..., : h * d].view(batch, 1, h, d).transpose(1, 2)
    k_new = qkv[..., h * d:(h + hkv) * d].view(batch, 1, hkv, d).transpose(1, 2)
    v_new = qkv[..., (h + hkv) * d:].view(batch, 1, hkv, d).transpose(1, 2)
    host_k, host_v, q_rot = [], [], torch.zeros(batch, h, 1, d)
    for b in range(batch):
        pos = torch.tensor([lengths[b]])
        q_rot[b] = _rope_host(q_all[b], pos, cos_h, sin_h).float()
        host_k.append(torch.cat([hist_k[b], _rope_host(k_new[b], pos, cos_h, sin_h)], dim=1))
        host_v.append(torch.cat([hist_v[b], v_new[b]], dim=1))
    k_all, v_all = padded(host_k, step.max_total), padded(host_v, step.max_total)
    dev_k, dev_v = cache.gather(0, step)
    assert torch.equal(dev_k.cpu().float(), k_all) and torch.equal(dev_v.cpu().float(), v_all)
    want = of.attention(q_rot, k_all, v_all, torch.tensor(lengths), torch.tensor(step.total), 0.125)
    got = out.view(batch, 1, h, d).transpose(1, 2).float().cpu()
    assert (got - want).abs().max().item() < 2e-2


def _parts_case(bs, lengths, h, hkv, hidden_dim, seed, max_kv_len=None, accumulate=True, tiled=True, nparts=4,
                attn_rows=None, extras=None):
    """A draft-style step (one new token per row, the norm finished inside) on
    two identical caches: rope_paged_attention (split -1) then linear(attn,
    wo) on the first; rope_paged_attention_parts then linear_attn_parts on
    the second (reading o_proj's weight in its tiled layout unless `tiled`
    is false; `nparts` partials per kv head; the folded rows to `attn_rows`
    when given).  Returns both outputs and both caches' gathered K/V; `extras`
    (a dict, when given) receives wo and the attention-only kernel's rows."""
    from lm.model import LlamaShape, rope_tables

    d, batch = 64, len(lengths)
    shape = LlamaShape(vocab_size=8, hidden_size=h * d, num_hidden_layers=1, num_attention_heads=h,
                       num_key_value_heads=hkv, intermediate_size=8, rope_theta=100000.0)
    cos, sin = (x.cuda() for x in rope_tables(shape, 2112))
    g = torch.Generator().manual_seed(seed)
    hist_k = [torch.randn(hkv, n, d, generator=g).to(torch.bfloat16) for n in lengths]
    hist_v = [torch.randn(hkv, n, d, generator=g).to(torch.bfloat16) for n in lengths]
    hidden = torch.randn(batch, 1, hidden_dim, generator=g).to(torch.bfloat16).cuda()
    qkv = torch.randn(batch, 1, (h + 2 * hkv) * d, generator=g).to(torch.bfloat16).cuda()
    wo = (torch.randn(hidden_dim, h * d, generator=g) * 0.05).to(torch.bfloat16).cuda()
    ids = list(range(batch))
    res = []
    for which in range(2):
        cache = make_cache(1, hkv, d, sum(n // bs + 3 for n in lengths) + 8, bs, torch.bfloat16, 11)
        for s_ in ids:
            cache.add(s_)
        step = cache.append(ids, lengths)
        cache.write(0, step, padded(hist_k, max(lengths)).to(torch.bfloat16).cuda(),
                    padded(hist_v, max(lengths)).to(torch.bfloat16).cuda())
        step = cache.append(ids, [1] * batch)
        kv_max = step.max_total if max_kv_len is None else max_kv_len
        out = hidden.clone() if accumulate else torch.zeros_like(hidden)
        if which == 0:
            attn = torch.zeros(batch, 1, h * d, dtype=torch.bfloat16, device="cuda")
            ops.rope_paged_attention(qkv.clone(), cos, sin, cache.k[0], cache.v[0], cache.table_tensor, step.meta,
                                     batch, 1, h, hkv, d, bs, 0.125, kv_max, attn, attn.stride(1), split_tokens=-1,
                                     norm_of=hidden, eps=1e-5)
            ops.linear(attn.view(batch, h * d), wo, out=out.view(batch, hidden_dim), accumulate=accumulate)
            if extras is not None:
                extras.update(wo=wo, attn=attn.view(batch, h * d))
        else:
            parts = ops.decode_parts_buffer(batch, h, "cuda", nparts)
            ops.rope_paged_attention_parts(qkv.clone(), cos, sin, cache.k[0], cache.v[0], cache.table_tensor,
                                           step.meta, batch, h, hkv, d, bs, 0.125, kv_max, parts, norm_of=hidden,
                                           eps=1e-5)
            ops.linear_attn_parts(parts, batch, h, ops.tile_weight(wo) if tiled else wo, out.view(batch, hidden_dim),
                                  accumulate=accumulate, attn_out=attn_rows)
        res.append((out, cache.gather(0, step)))
    return res


@pytest.mark.parametrize("bs", [16, 32])
@pytest.mark.parametrize("lengths", [[300], [1], [63], [64], [1000], [2047], [300, 37, 1]])
@pytest.mark.parametrize("heads,hidden_dim", [((9, 3), 576), ((4, 2), 256), ((8, 1), 512), ((32, 32), 2048)])
def test_decode_parts_then_projection_equal_attention_then_linear(bs, lengths, heads, hidden_dim):
    """The draft step through split partials (four one-wave workgroups per
    kv head, folded by the o_proj launch) has the bits of the attention-only
    decode kernel followed by specdec_linear: the residual row after o_proj
    and the pools (the appended token) are equal bit for bit."""
    (ref, kv_ref), (got, kv_got) = _parts_case(bs, lengths, heads[0], heads[1], hidden_dim, seed=bs + heads[0])
    assert torch.equal(got, ref)
    assert torch.equal(kv_got[0], kv_ref[0]) and torch.equal(kv_got[1], kv_ref[1])


def test_decode_parts_without_accumulate_equal_plain_projection():
    (ref, _), (got, _) = _parts_case(16, [300, 5], 9, 3, 576, seed=3, accumulate=False)
    assert torch.equal(got, ref)


@pytest.mark.parametrize("heads,hidden_dim", [((9, 3), 576), ((32, 32), 2048)])
def test_decode_parts_with_row_major_weight(heads, hidden_dim):
    (ref, _), (got, _) = _parts_case(16, [300, 37], heads[0], heads[1], hidden_dim, seed=4, tiled=False)
    assert torch.equal(got, ref)


@pytest.mark.parametrize("nparts", [8, 16])
@pytest.mark.parametrize("lengths", [[300], [1], [1000, 64], [2047]])
def test_decode_parts_of_other_counts(nparts, lengths):
    """More partials per kv head (8 or 16, one per 64-token step): the
    folded attention rows agree with the attention-only kernel's to bf16
    rounding (another fold order), o_proj of them has specdec_linear's bits
    on those rows, and the pools are the same bit for bit."""
    h, hkv, hidden_dim = 9, 3, 576
    batch = len(lengths)
    rows = torch.zeros(batch, h * 64, dtype=torch.bfloat16, device="cuda")
    extras = {}
    (ref, kv_ref), (got, kv_got) = _parts_case(16, lengths, h, hkv, hidden_dim, seed=nparts + lengths[0],
                                               accumulate=False, nparts=nparts, attn_rows=rows, extras=extras)
    assert (rows.float() - extras["attn"].float()).abs().max().item() < 2e-2
    assert torch.equal(got.view(batch, hidden_dim), ops.linear(rows, extras["wo"]))
    assert torch.equal(kv_got[0], kv_ref[0]) and torch.equal(kv_got[1], kv_ref[1])


def test_decode_parts_counts_follow_the_context():
    assert [ops.decode_parts_count(n) for n in (1, 256, 257, 300, 512, 1024, 2048)] == [4, 4, 8, 8, 8, 8, 8]
    with pytest.raises(ValueError):
        ops.decode_parts_buffer(1, 9, "cuda", 5)


def test_decode_parts_rows_beyond_max_kv_len_are_nan():
    """A row whose cached length exceeds the call's max_kv_len (a broken
    contract) gets NaN, as from the attention-only kernel."""
    for max_kv_len in (64, 300):  # 300: one key short of the row's 301, within its last 64-key step
        (ref, _), (got, _) = _parts_case(16, [300], 9, 3, 576, seed=5, max_kv_len=max_kv_len)
        assert torch.isnan(ref.float()).all() and torch.isnan(got.float()).all()


def test_decode_parts_reject_other_shapes():
    parts = ops.decode_parts_buffer(17, 9, "cuda")
    wo = torch.zeros(576, 576, dtype=torch.bfloat16, device="cuda")
    out = torch.zeros(17, 576, dtype=torch.bfloat16, device="cuda")
    with pytest.raises(NotImplementedError):  # more than 16 rows
        ops.linear_attn_parts(parts, 17, 9, wo, out)
    with pytest.raises(ValueError):  # w of another inner size
        ops.linear_attn_parts(parts[:1], 1, 9, wo[:, :512], out[:1])
    assert not ops.decode_parts_fit(torch.bfloat16, 1, 1, 9, 3, 64, 16, 4096, -1)
    assert not ops.decode_parts_fit(torch.bfloat16, 1, 5, 9, 3, 64, 16, 512, -1)


def test_input_norm_in_attention_rejects_other_shapes():
    cache, step, q, _ = _filled(1, [40], 0)
    h = torch.zeros(1, 20, 64, dtype=torch.bfloat16, device="cuda")
    qkv = torch.zeros(1, 20, 96 * 64, dtype=torch.bfloat16, device="cuda")
    cos = sin = torch.zeros(128, 32, device="cuda")
    out = torch.zeros(1, 20, 32 * 64, dtype=torch.bfloat16, device="cuda")
    with pytest.raises(ValueError, match="width"):
        ops.rope_paged_attention(qkv, cos, sin, cache.k[0], cache.v[0], cache.table_tensor, step.meta, 1, 20, 32, 32,
                                 64, 16, 0.125, step.max_total, out, out.stride(1), norm_of=h, eps=1e-5)


def _rope_host(x: torch.Tensor, pos: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """transformers' rotate_half RoPE of x [..., T, 64] (bf16) at positions
    pos [T], in fp32 with every product and sum rounded on its own, then
    rounded to bf16 -- where the kernel rounds a rotated q or k."""
    x = x.float()
    c, s = cos[pos], sin[pos]  # [T, 32]
    x1, x2 = x[..., :32], x[..., 32:]
    return torch.cat([x1 * c - x2 * s, x2 * c + x1 * s], dim=-1).to(torch.bfloat16)


@pytest.mark.parametrize("width,bs", [(256, 16), (1024, 16), (256, 32)])
@pytest.mark.parametrize("heads", [(32, 32), (9, 3)])
@pytest.mark.parametrize("past", [[0, 0], [100, 0]])
def test_bf16_prefill_matches_oracle(width, bs, heads, past):
    """A prompt-sized append (256 or 1024 new tokens, right-padded rows of
    different lengths, from an empty cache or after a cached chunk that
    ends inside a 16-position group) through the fused RoPE + append +
    attention launch, in bf16, with blocks of 16 and 32, against the
    reference's prefill step restated on the host (lm/forward.py:40-49,
    53, 60-63): RoPE of q and k, the new K/V appended after the cached
    ones, causal SDPA.  The pool must hold the host's rotated k and v bit
    for bit."""
    from lm.model import LlamaShape, rope_tables

    h, hkv = heads
    d, batch = 64, 2
    n_new = [width, width - 37]
    theta = 130000.0 if h == 32 else 100000.0
    shape = LlamaShape(vocab_size=8, hidden_size=h * d, num_hidden_layers=1, num_attention_heads=h,
                       num_key_value_heads=hkv, intermediate_size=8, rope_theta=theta)
    cos_h, sin_h = rope_tables(shape, 2048)
    cos, sin = cos_h.cuda(), sin_h.cuda()
    g = torch.Generator().manual_seed(width + h + past[0])
    cache = make_cache(1, hkv, d, sum((p + n) // bs + 2 for p, n in zip(past, n_new)) + 8, bs, torch.bfloat16, 5)
    ids = list(range(batch))
    for s in ids:
        cache.add(s)
    hist_k = [torch.randn(hkv, p, d, generator=g).to(torch.bfloat16) for p in past]
    hist_v = [torch.randn(hkv, p, d, generator=g).to(torch.bfloat16) for p in past]
    if max(past) > 0:
        step = cache.append(ids, past)
        cache.write(0, step, padded(hist_k, max(past)).to(torch.bfloat16).cuda(),
                    padded(hist_v, max(past)).to(torch.bfloat16).cuda())
    step = cache.append(ids, n_new)
    qkv = torch.randn(batch, width, (h + 2 * hkv) * d, generator=g).to(torch.bfloat16)
    out = torch.zeros(batch, width, h * d, dtype=torch.bfloat16, device="cuda")
    x = qkv.cuda()
    ops.rope_paged_attention(x, cos, sin, cache.k[0], cache.v[0], cache.table_tensor, step.meta, batch, width, h, hkv,
                             d, bs, 0.125, step.max_total, out, out.stride(1))
    # host: rotated q/k of the real tokens, K/V after the cached chunk
    q_all = qkv[..., : h * d].view(batch, width, h, d).transpose(1, 2)
    k_new = qkv[..., h * d:(h + hkv) * d].view(batch, width, hkv, d).transpose(1, 2)
    v_new = qkv[..., (h + hkv) * d:].view(batch, width, hkv, d).transpose(1, 2)
    host_k, host_v, q_rot = [], [], torch.zeros(batch, h, width, d)
    for b in range(batch):
        pos = torch.arange(past[b], past[b] + n_new[b])
        q_rot[b, :, : n_new[b]] = _rope_host(q_all[b, :, : n_new[b]], pos, cos_h, sin_h).float()
        host_k.append(torch.cat([hist_k[b], _rope_host(k_new[b, :, : n_new[b]], pos, cos_h, sin_h)], dim=1))
        host_v.append(torch.cat([hist_v[b], v_new[b, :, : n_new[b]]], dim=1))
    k_all, v_all = padded(host_k, step.max_total), padded(host_v, step.max_total)
    dev_k, dev_v = cache.gather(0, step)
    assert torch.equal(dev_k.cpu().float(), k_all) and torch.equal(dev_v.cpu().float(), v_all)
    want = of.attention(q_rot, k_all, v_all, torch.tensor(past), torch.tensor(step.total), 0.125)
    got = out.view(batch, width, h, d).transpose(1, 2).float().cpu()
    for b in range(batch):
        err = (got[b, :, : n_new[b]] - want[b, :, : n_new[b]]).abs()
        assert err.max().item() < 2e-2 and err.mean().item() < 2e-3, (b, err.max().item(), err.mean().item())


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("t_new,max_kv_len", [(5, 1030), (5, 2600), (5, 4004), (20, 4010)])
def test_rows_beyond_max_kv_len_get_nan(dtype, t_new, max_kv_len):
    """A caller passing a max_kv_len below a row's key count breaks the
    contract: that row's output is NaN (not left stale, and no key past
    max_kv_len is read), the other rows are exact.  1030 keys: the
    one-workgroup grid; 2600: split partials and the combine launch; 4004:
    one key short of the row's 4005, within the last split; 20 new tokens:
    the prompt-sized kernel (bf16), every query tile of the row past 4010."""
    d, h, hkv, bs = 64, 8, 8, 16
    lengths = [100, 4000]
    g = torch.Generator().manual_seed(9)
    cache = make_cache(1, hkv, d, sum(L // bs + 2 for L in lengths) + 8, bs, dtype, 9)
    for s in (0, 1):
        cache.add(s)
    step = cache.append([0, 1], lengths)
    kh = torch.randn(2, hkv, max(lengths), d, generator=g).to(dtype)
    vh = torch.randn(2, hkv, max(lengths), d, generator=g).to(dtype)
    cache.write(0, step, kh.cuda(), vh.cuda())
    step = cache.append([0, 1], [t_new, t_new])
    kn = torch.randn(2, hkv, t_new, d, generator=g).to(dtype)
    vn = torch.randn(2, hkv, t_new, d, generator=g).to(dtype)
    cache.write(0, step, kn.cuda(), vn.cuda())
    q = torch.randn(2, t_new, h * d, generator=g).to(dtype).cuda()
    out = torch.zeros(2, t_new, h * d, dtype=dtype, device="cuda")
    ops.paged_attention(q, q.stride(1), cache.k[0], cache.v[0], cache.table_tensor, step.meta, 2, t_new, h, hkv, d,
                        bs, d ** -0.5, max_kv_len, out, out.stride(1))
    got = out.float().cpu()
    assert bool(torch.isnan(got[1]).all())
    k0 = torch.cat([kh[0, :, :100], kn[0]], dim=1).float()[None]
    v0 = torch.cat([vh[0, :, :100], vn[0]], dim=1).float()[None]
    want = of.attention(q[:1].view(1, t_new, h, d).transpose(1, 2).float().cpu(), k0, v0, torch.tensor([100]),
                        torch.tensor([100 + t_new]), d ** -0.5)
    tol = 2e-2 if dtype == torch.bfloat16 else 2e-5
    assert (got[0].view(t_new, h, d).transpose(0, 1) - want[0]).abs().max().item() < tol


def test_short_token_buffers_are_refused_before_launch():
    """q, qkv and out must hold batch x width token rows at the strides the
    call is given: a shorter buffer, or a stride shorter than a token's heads,
    is refused on the host (a kernel would read or write past it)."""
    d, h, hkv, bs, t_new = 64, 4, 4, 16, 5
    cache = make_cache(1, hkv, d, 16, bs, torch.bfloat16, 3)
    cache.add(0)
    cache.append([0], [32])
    step = cache.append([0], [t_new])
    q = torch.zeros(1, t_new, h * d, dtype=torch.bfloat16, device="cuda")
    out = torch.zeros_like(q)
    args = (cache.k[0], cache.v[0], cache.table_tensor, step.meta, 1, t_new, h, hkv, d, bs, 0.125, 37)
    # (a view into a larger buffer is memory the kernel may use: the short
    # buffers are tensors of their own)
    short_q = torch.zeros(1, 4, h * d, dtype=torch.bfloat16, device="cuda")
    with pytest.raises(ValueError, match="q holds"):
        ops.paged_attention(short_q, short_q.stride(1), *args, out, out.stride(1))
    short_out = torch.zeros(1, 3, h * d, dtype=torch.bfloat16, device="cuda")
    with pytest.raises(ValueError, match="out holds"):
        ops.paged_attention(q, q.stride(1), *args, short_out, short_out.stride(1))
    with pytest.raises(ValueError, match="token stride"):
        ops.paged_attention(q, h * d - 64, *args, out, out.stride(1))
    with pytest.raises(ValueError, match="q holds"):
        ops.paged_attention_static(short_q, short_q.stride(1), *args, out, out.stride(1))
    short_qkv = torch.zeros(1, 2, (h + 2 * hkv) * d, dtype=torch.bfloat16, device="cuda")
    cos = torch.ones(64, d // 2, device="cuda")
    sin = torch.zeros(64, d // 2, device="cuda")
    with pytest.raises(ValueError, match="qkv holds"):
        ops.rope_paged_attention(short_qkv, cos, sin, *args, out, out.stride(1))
    with pytest.raises(ValueError, match="qkv holds"):
        ops.rope_append(short_qkv, h, hkv, d, cos, sin, step.meta, 1, t_new, cache.table_tensor, bs, cache.k[0],
                        cache.v[0])
    # the same buffers at full length run
    ops.paged_attention(q, q.stride(1), *args, out, out.stride(1))
    torch.cuda.synchronize()
