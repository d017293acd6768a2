"""Device allocator, block tables and slot maps vs the reference semantics."""
import math
import random

import pytest
import torch

import oracle.kv as okv
from cache.kv import KVCache
from cache.paged import BlockAllocator, BlockTable, OutOfBlocks
from helpers import golden

pytestmark = pytest.mark.gpu
DEV = "cuda"


def test_exhaustion_raises():
    allocator = BlockAllocator(3, DEV)
    assert [allocator.allocate() for _ in range(3)] == [0, 1, 2]
    with pytest.raises(OutOfBlocks):
        allocator.allocate()


def test_double_free_and_foreign_free_raise():
    allocator = BlockAllocator(2, DEV)
    block = allocator.allocate()
    allocator.free(block)
    with pytest.raises(ValueError):
        allocator.free(block)
    with pytest.raises(ValueError):
        allocator.free(99)
    allocator.check()


def test_lifo_order():
    allocator = BlockAllocator(5, DEV)
    a, b, c = allocator.allocate(), allocator.allocate(), allocator.allocate()
    allocator.free(b)
    allocator.free(a)
    assert allocator.allocate() == a and allocator.allocate() == b and allocator.allocate() == 3
    assert allocator.peak_used == 4


def test_failed_grow_changes_nothing():
    allocator = BlockAllocator(3, DEV)
    table = BlockTable(device=DEV)
    table.grow_to(8, allocator, block_size=4)
    with pytest.raises(OutOfBlocks):
        table.grow_to(13, allocator, block_size=4)
    assert table.length == 8 and len(table.blocks) == 2 and allocator.num_free == 1
    allocator.check()


@pytest.mark.parametrize(("length", "blocks"), [(9, 3), (8, 2), (5, 2), (4, 1), (1, 1), (0, 0)])
def test_shrink_keeps_ceil_length_over_block_size(length, blocks):
    allocator = BlockAllocator(4, DEV)
    table = BlockTable(device=DEV)
    table.grow_to(9, allocator, block_size=4)
    table.shrink_to(length, allocator, block_size=4)
    assert len(table.blocks) == blocks
    assert allocator.num_free == 4 - blocks
    allocator.check()


def test_slot_arithmetic():
    table = BlockTable(blocks=[7, 2], length=6, device=DEV)
    assert table.slots(0, 6, block_size=4).tolist() == [28, 29, 30, 31, 8, 9]
    assert table.slots(3, 5, block_size=4).tolist() == [31, 8]


def _cache(block_size, num_blocks):
    return KVCache(n_layers=2, n_kv_heads=2, head_dim=8, num_blocks=num_blocks, block_size=block_size,
                   dtype=torch.float32, device=DEV)


def test_fragmentation_hand_case():
    cache = _cache(4, 8)
    for seq_id, length in enumerate([5, 8, 1]):
        cache.add(seq_id)
        cache.append([seq_id], [length])
    stats = cache.stats()
    assert stats.blocks_in_use == 5 and stats.slots_allocated == 20 and stats.slots_used == 14
    assert stats.waste == pytest.approx(0.3)
    assert stats.bytes_per_slot == 256 and stats.bytes_in_use == 20 * 256


def test_peak_survives_free():
    cache = _cache(4, 8)
    cache.add(0)
    cache.append([0], [12])
    cache.free(0)
    assert cache.stats().blocks_in_use == 0
    assert cache.stats().peak_blocks_in_use == 3


def test_random_operations_keep_free_list_consistent():
    rng = random.Random(0)
    bs = 3
    cache = _cache(bs, 40)
    live, next_id = [], 0
    for i in range(600):
        op = rng.random()
        if op < 0.2 or not live:
            cache.add(next_id)
            live.append(next_id)
            next_id += 1
        elif op < 0.6:
            try:
                cache.append([rng.choice(live)], [rng.randint(1, 7)])
            except OutOfBlocks:
                pass
        elif op < 0.85:
            s = rng.choice(live)
            cache.truncate(s, rng.randint(0, cache.length(s)))
        else:
            cache.free(live.pop(rng.randrange(len(live))))
        if i % 20 == 0:
            cache.allocator.check()
            owned = [b for t in cache.tables.values() for b in t.blocks]
            assert len(owned) == len(set(owned)) == cache.allocator.num_used
            for t in cache.tables.values():
                assert len(t.blocks) == math.ceil(t.length / bs)


@pytest.mark.parametrize("run", range(4))
def test_golden_block_ids_and_free_list_order(run):
    """Replays the reference's seeded op sequences; block ids of every table,
    the free-list order and the stats match after every operation."""
    data = golden("paged_ops.json")["runs"][run]
    bs, nb = data["block_size"], data["num_blocks"]
    cache = KVCache(n_layers=1, n_kv_heads=1, head_dim=2, num_blocks=nb, block_size=bs, dtype=torch.float32,
                    device=DEV)
    for entry in data["log"]:
        op = entry["op"]
        if op[0] == "add":
            cache.add(op[1])
        elif op[0] == "append":
            if op[3] == "ok":
                cache.append(op[1], op[2])
            else:
                with pytest.raises(OutOfBlocks):
                    cache.append(op[1], op[2])
        elif op[0] == "truncate":
            cache.truncate(op[1], op[2])
        else:
            cache.free(op[1])
        cache.flush()
        got_tables = {str(s): [t.blocks, t.length] for s, t in cache.tables.items()}
        assert got_tables == entry["tables"], op
        free = cache.allocator._stack[: cache.allocator._dev_top].cpu().tolist()
        assert free == entry["free"], op
        st = cache.stats()
        assert [st.blocks_in_use, st.peak_blocks_in_use, st.slots_used] == entry["stats"]
        assert cache.allocator.peak_used == entry["peak"]


@pytest.mark.parametrize("bs", [1, 3, 4, 16])
def test_slot_map_matches_reference_append(bs):
    """SlotMap write/write_index/read/past/total equal the reference's, for a
    padded batch over several rounds with rollbacks in between."""
    ours = KVCache(1, 1, 8, 64, bs, torch.float32, DEV)
    ref = okv.KVCache(1, 1, 8, 64, bs, torch.float32)
    for s in range(3):
        ours.add(s)
        ref.add(s)
    rng = random.Random(bs)
    for r in range(12):
        ids = [0, 1, 2]
        n_new = [rng.randint(1, 9) for _ in ids]
        want = ref.append(ids, n_new)
        got = ours.append(ids, n_new).slot_map()
        for f in ("write", "write_index", "read", "past", "total"):
            assert getattr(got, f).cpu().tolist() == getattr(want, f).tolist(), (r, f)
        for s in ids:
            keep = rng.randint(0, ref.length(s))
            ref.truncate(s, keep)
            ours.truncate(s, keep)
