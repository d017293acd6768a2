"""specdec_paged_attention_static -- verify attention whose split partials
live in the library's own per-GPU buffer -- against specdec_paged_attention
with a caller workspace, both through the C ABI.  The two run the same
kernels with the same arithmetic, so the outputs must be equal bit for bit:
on two calls in a row (the second smaller, so it reads a buffer the first
left full of its own partials), in bf16 and fp32, and an oversized call is
refused before anything is launched."""
import pytest
import torch

from cache.kv import KVCache
from specdec import _lib, ops

pytestmark = pytest.mark.gpu
D = 64


def shuffled_cache(hkv, num_blocks, bs, dtype, seed):
    """One-layer cache whose blocks come off the free list in a seeded random order."""
    cache = KVCache(1, hkv, D, num_blocks, bs, dtype, "cuda")
    perm = torch.randperm(num_blocks, generator=torch.Generator().manual_seed(seed))
    cache.add(-1)
    cache.append([-1], [num_blocks * bs])
    cache.table_tensor[cache.tables[-1].row, :num_blocks] = perm.to(torch.int32).cuda()
    cache.free(-1)
    cache.flush()
    return cache


def both_entry_points(lengths, h, hkv, dtype, seed, t_new=5, bs=16):
    """Fill a cache to `lengths`, append t_new tokens per row, run the verify
    attention through both entry points; returns (static, workspace) outputs
    and the number of split partials the call needed."""
    batch = len(lengths)
    nb = sum(-(-(n + t_new) // bs) for n in lengths) + 4
    cache = shuffled_cache(hkv, nb, bs, dtype, seed)
    ids = list(range(batch))
    for s in ids:
        cache.add(s)
    g = torch.Generator(device="cuda").manual_seed(seed)
    cache.append(ids, lengths)
    cache.k.normal_(generator=g)
    cache.v.normal_(generator=g)
    step = cache.append(ids, [t_new] * batch)
    q = torch.randn(batch, t_new, h * D, generator=g, device="cuda").to(dtype)
    args = (q, q.stride(1), cache.k[0], cache.v[0], cache.table_tensor, step.meta, batch, t_new, h, hkv, D, bs,
            D ** -0.5, step.max_total)
    ref = torch.full_like(q, float("nan"))
    got = torch.full_like(q, float("nan"))
    ops.paged_attention(*args, ref, ref.stride(1), ops.AttentionWorkspace(q.device))
    ops.paged_attention_static(*args, got, got.stride(1))
    torch.cuda.synchronize()
    need = ops.attention_workspace_floats(batch, t_new, h, hkv, D, step.max_total)
    return got, ref, need


def test_two_calls_in_a_row_equal_the_workspace_entry_point():
    # call 1: batch 4 at ~4096 keys -- 128 (row, head) units of 8 splits,
    # 4-wave split kernel + combine, 1.06 M partial floats
    print("[case] static attention bf16 B=4 L~4096", flush=True)
    got, ref, need = both_entry_points([4096, 4093, 4090, 4087], 32, 32, torch.bfloat16, seed=1)
    assert 0 < need <= _lib.STATIC_PARTIAL_FLOATS
    assert not torch.isnan(ref).any()
    assert torch.equal(got, ref)
    # call 2, smaller: batch 1 at 2500 keys (5 splits: partials + combine)
    print("[case] static attention bf16 B=1 L=2500", flush=True)
    got, ref, need = both_entry_points([2500], 32, 32, torch.bfloat16, seed=2)
    assert 0 < need
    assert not torch.isnan(ref).any()
    assert torch.equal(got, ref)


def test_fp32_and_gqa_calls_equal_the_workspace_entry_point():
    print("[case] static attention fp32 GQA 8/4 B=3", flush=True)
    got, ref, _ = both_entry_points([1500, 900, 1201], 8, 4, torch.float32, seed=3)
    assert torch.equal(got, ref)
    print("[case] static attention fp32 GQA 8/4 B=1 (smaller)", flush=True)
    got, ref, _ = both_entry_points([700], 8, 4, torch.float32, seed=4)
    assert torch.equal(got, ref)


def test_call_without_partials_needs_no_buffer():
    # 2048 keys: one 16-wave workgroup per unit folds its four splits in LDS
    print("[case] static attention bf16 B=2 L=1500 (no partials)", flush=True)
    got, ref, _ = both_entry_points([1500, 1400], 32, 32, torch.bfloat16, seed=5)
    assert torch.equal(got, ref)


def test_oversized_call_is_refused_before_launch():
    """Batch 8 at 8192 keys needs 256 units x 17 splits of partials (4.5 M
    floats): refused with SPECDEC_ENOSCRATCH, nothing launched, output untouched."""
    dev = torch.device("cuda")
    q = torch.zeros(8, 5, 32 * D, dtype=torch.bfloat16, device=dev)
    out = torch.full_like(q, 7.0)
    pool = torch.zeros(4, 32, 16, D, dtype=torch.bfloat16, device=dev)
    tables = torch.zeros(8, 4, dtype=torch.int32, device=dev)
    meta = torch.zeros(3, 8, dtype=torch.int32, device=dev)
    with pytest.raises(ops.KernelError, match="static buffer"):
        ops.paged_attention_static(q, q.stride(1), pool, pool, tables, meta, 8, 5, 32, 32, D, 16, 0.125, 8197, out,
                                   out.stride(1))
    torch.cuda.synchronize()
    assert bool((out == 7.0).all())
