"""Oracle of cache/kv.py (test infrastructure, see oracle/__init__.py)."""
from dataclasses import dataclass

import torch

from oracle.paged import BlockAllocator, BlockTable, FragmentationStats


@dataclass(frozen=True)
class SlotMap:
    """cache/kv.py:9-15"""
    write: torch.Tensor
    write_index: torch.Tensor
    read: torch.Tensor
    past: torch.Tensor
    total: torch.Tensor


class KVCache:
    """cache/kv.py:18-127: pool [L, NB*bs, Hkv, d] on the CPU."""

    def __init__(self, n_layers, n_kv_heads, head_dim, num_blocks, block_size, dtype, device="cpu"):
        self.block_size = block_size
        self.device = torch.device(device)
        self.allocator = BlockAllocator(num_blocks)
        shape = (n_layers, num_blocks * block_size, n_kv_heads, head_dim)
        self.k = torch.zeros(shape, dtype=dtype, device=self.device)
        self.v = torch.zeros(shape, dtype=dtype, device=self.device)
        self.tables: dict[int, BlockTable] = {}
        self.bytes_per_slot = 2 * n_layers * n_kv_heads * head_dim * self.k.element_size()

    @classmethod
    def for_model(cls, config, num_blocks, block_size, dtype, device="cpu"):
        head_dim = getattr(config, "head_dim", None) or config.hidden_size // config.num_attention_heads
        return cls(config.num_hidden_layers, config.num_key_value_heads, head_dim, num_blocks, block_size, dtype,
                   device)

    def add(self, seq_id):
        if seq_id in self.tables:
            raise ValueError(f"sequence {seq_id} already present")
        self.tables[seq_id] = BlockTable()

    def free(self, seq_id):
        self.tables[seq_id].shrink_to(0, self.allocator, self.block_size)
        del self.tables[seq_id]

    def length(self, seq_id):
        return self.tables[seq_id].length

    def append(self, seq_ids, n_new):
        """cache/kv.py:79-99"""
        width = max(n_new)
        past = [self.tables[s].length for s in seq_ids]
        for seq_id, n in zip(seq_ids, n_new):
            table = self.tables[seq_id]
            table.grow_to(table.length + n, self.allocator, self.block_size)
        total = [p + n for p, n in zip(past, n_new)]
        write = torch.cat([self.tables[s].slots(p, t, self.block_size) for s, p, t in zip(seq_ids, past, total)])
        write_index = torch.cat([b * width + torch.arange(n) for b, n in enumerate(n_new)])
        read = torch.zeros(len(seq_ids), max(total), dtype=torch.long)
        for b, (seq_id, t) in enumerate(zip(seq_ids, total)):
            read[b, :t] = self.tables[seq_id].slots(0, t, self.block_size)

        def put(x):
            return torch.as_tensor(x, dtype=torch.long).to(self.device)

        return SlotMap(put(write), put(write_index), put(read), put(past), put(total))

    def write(self, layer, slots, k, v):
        """cache/kv.py:101-106"""
        b, h, t, d = k.shape
        rows = slots.write_index
        self.k[layer][slots.write] = k.transpose(1, 2).reshape(b * t, h, d)[rows]
        self.v[layer][slots.write] = v.transpose(1, 2).reshape(b * t, h, d)[rows]

    def gather(self, layer, slots):
        """cache/kv.py:108-112"""
        return self.k[layer][slots.read].transpose(1, 2), self.v[layer][slots.read].transpose(1, 2)

    def truncate(self, seq_id, length):
        """cache/kv.py:114-118"""
        self.tables[seq_id].shrink_to(length, self.allocator, self.block_size)

    def stats(self):
        return FragmentationStats(self.block_size, self.bytes_per_slot, self.allocator.num_used,
                                  self.allocator.peak_used, sum(t.length for t in self.tables.values()))
