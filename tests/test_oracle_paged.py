"""Pins oracle.paged / oracle.kv against the reference's literals and the
golden op sequences the reference produced."""
import pytest
import torch

import oracle.kv as okv
from helpers import golden
from oracle.paged import BlockAllocator, BlockTable, OutOfBlocks


def test_literals():
    a = BlockAllocator(3)
    assert [a.allocate() for _ in range(3)] == [0, 1, 2]
    with pytest.raises(OutOfBlocks):
        a.allocate()
    t = BlockTable(blocks=[7, 2], length=6)
    assert t.slots(0, 6, 4).tolist() == [28, 29, 30, 31, 8, 9]
    a = BlockAllocator(3)
    t = BlockTable()
    t.grow_to(8, a, 4)
    with pytest.raises(OutOfBlocks):
        t.grow_to(13, a, 4)
    assert t.length == 8 and len(t.blocks) == 2 and a.num_free == 1


@pytest.mark.parametrize("run", range(4))
def test_golden_op_sequences(run):
    data = golden("paged_ops.json")["runs"][run]
    cache = okv.KVCache(1, 1, 2, data["num_blocks"], data["block_size"], torch.float32)
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
        assert {str(s): [t.blocks, t.length] for s, t in cache.tables.items()} == entry["tables"]
        assert cache.allocator.free_list() == entry["free"]
        st = cache.stats()
        assert [st.blocks_in_use, st.peak_blocks_in_use, st.slots_used] == entry["stats"]
