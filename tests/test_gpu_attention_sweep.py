"""A seeded sweep of verify-attention call shapes against the oracle's
attention: ragged batches of 1-9 rows with 1-3000 cached keys each, 1-33 new
tokens per row (past 16 the prompt kernel), GQA groups 1-4, block sizes the
kernels specialise (16, 32) and ones they take generically, bf16 and fp32,
two rounds each with rollback -- the shapes the parametrised tests leave
between their cases."""
import random

import pytest
import torch

from specdec import ops
from test_gpu_attention import make_cache, run_case

pytestmark = pytest.mark.gpu


def _cases(n=48, seed=2024):
    rng = random.Random(seed)
    out = []
    for i in range(n):
        dtype = rng.choice([torch.bfloat16, torch.float32])
        h, hkv = rng.choice([(32, 32), (8, 2), (9, 3), (4, 4), (16, 4), (12, 3)])
        bs = rng.choice([4, 16, 16, 32]) if dtype == torch.bfloat16 else rng.choice([1, 3, 8, 16, 32])
        batch = rng.randint(1, 9)
        t_new = rng.choice([1, 2, 5, 5, 9, 16, 17, 33])
        lengths = [rng.randint(1, 3000) for _ in range(batch)]
        out.append(pytest.param(batch, lengths, h, hkv, bs, dtype, t_new, 7000 + i,
                                id=f"{i}-b{batch}-t{t_new}-h{h}x{hkv}-bs{bs}-{str(dtype)[6:]}"))
    return out


@pytest.mark.parametrize("batch,lengths,h,hkv,bs,dtype,t_new,seed", _cases())
def test_random_shapes_match_oracle(batch, lengths, h, hkv, bs, dtype, t_new, seed):
    for got, want in run_case(batch, lengths, h, hkv, bs, dtype, t_new, seed):
        if dtype == torch.bfloat16:
            err = (got - want).abs().max().item()
            assert err < 2e-2, err
        else:
            assert torch.allclose(got, want, atol=2e-5, rtol=1e-5), (got - want).abs().max()


def _fused_cases(n=24, seed=77):
    rng = random.Random(seed)
    out = []
    for i in range(n):
        dtype = rng.choice([torch.bfloat16, torch.float32])
        h, hkv = rng.choice([(32, 32), (8, 2), (9, 3), (4, 4), (16, 4)])
        bs = rng.choice([4, 16, 16, 32])
        batch = rng.choice([1, 2, 5, 9])
        t_new = rng.choice([1, 3, 5, 5, 9, 16, 17, 40])
        lengths = [rng.choice([0, rng.randint(1, 3000)]) for _ in range(batch)]
        out.append(pytest.param(batch, lengths, h, hkv, bs, dtype, t_new, 9000 + i,
                                id=f"{i}-b{batch}-t{t_new}-h{h}x{hkv}-bs{bs}-{str(dtype)[6:]}"))
    return out


@pytest.mark.parametrize("batch,lengths,h,hkv,bs,dtype,t_new,seed", _fused_cases())
def test_random_shapes_fused_append_equals_separate_kernels(batch, lengths, h, hkv, bs, dtype, t_new, seed):
    """rope_paged_attention (RoPE and the append inside the attention launch)
    == rope_append followed by paged_attention, output and pools bit for bit,
    over the sweep's shapes (rows without history included)."""
    from lm.model import LlamaShape, rope_tables

    d = 64
    shape = LlamaShape(vocab_size=8, hidden_size=h * d, num_hidden_layers=1, num_attention_heads=h,
                       num_key_value_heads=hkv, intermediate_size=8, rope_theta=10000.0)
    cos, sin = (x.cuda() for x in rope_tables(shape, 4096))
    g = torch.Generator().manual_seed(seed)
    nb = sum((n + t_new + bs) // bs + 1 for n in lengths) + 8
    ids = list(range(batch))
    hist = [torch.randn(batch, hkv, max(max(lengths), 1), d, generator=g).to(dtype).cuda() for _ in range(2)]
    qkv = torch.randn(batch, t_new, (h + 2 * hkv) * d, generator=g).to(dtype).cuda()
    outs = []
    for which in range(2):
        cache = make_cache(1, hkv, d, nb, bs, dtype, seed)
        for s_ in ids:
            cache.add(s_)
        step = cache.append(ids, lengths)
        if max(lengths) > 0:
            cache.write(0, step, hist[0], hist[1])
        step = cache.append(ids, [t_new] * batch)
        out = torch.zeros(batch, t_new, h * d, dtype=dtype, device="cuda")
        x = qkv.clone()
        if which == 0:
            ops.rope_append(x, h, hkv, d, cos, sin, step.meta, batch, t_new, cache.table_tensor, bs, cache.k[0],
                            cache.v[0])
            ops.paged_attention(x, x.stride(1), cache.k[0], cache.v[0], cache.table_tensor, step.meta, batch, t_new,
                                h, hkv, d, bs, 0.125, step.max_total, out, out.stride(1))
        else:
            ops.rope_paged_attention(x, cos, sin, cache.k[0], cache.v[0], cache.table_tensor, step.meta, batch, t_new,
                                     h, hkv, d, bs, 0.125, step.max_total, out, out.stride(1))
        k_all, v_all = cache.gather(0, step)
        outs.append((out, k_all, v_all))
    for a, b in zip(outs[0], outs[1]):
        assert torch.equal(a, b)
