"""Paged K/V pool on the GPU (reference: cache/kv.py:9-127).

Pool layout per layer (chosen so one (block, head) tile is contiguous):
    k[layer]: [num_blocks, n_kv_heads, block_size, head_dim]
    v[layer]: [num_blocks, n_kv_heads, head_dim, block_size]
Block ids come from the device allocator of cache.paged; one `append` is one
block-plan launch (queued rollbacks pushed, then growth popped) and one small
host-to-device copy of the per-row metadata the kernels read.  Rollback
(`truncate`) and `free` only queue their pushes, so the per-row calls of the
round loop cost no launch; the queue is applied, in call order, by the next
append or by anything that reads block ids.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

from cache.paged import (BlockAllocator, BlockTable, FragmentationStats, OutOfBlocks, _gpu_device, _TableStore,
                         _upload_i32)
from specdec import ops


@dataclass(frozen=True)
class SlotMap:
    """The reference's slot map (cache/kv.py:9-15), all int64 on the device."""

    write: torch.Tensor
    write_index: torch.Tensor
    read: torch.Tensor
    past: torch.Tensor
    total: torch.Tensor


@dataclass(frozen=True)
class PagedStep:
    """What the kernels of one forward need: `meta` int32 [3, B] on the device
    (table row, past length, new tokens per row) and the host copies."""

    cache: "KVCache"
    meta: torch.Tensor
    rows: list[int]
    past: list[int]
    n_new: list[int]
    width: int

    @property
    def batch(self) -> int:
        return len(self.rows)

    @property
    def total(self) -> list[int]:
        return [p + n for p, n in zip(self.past, self.n_new)]

    @property
    def max_total(self) -> int:
        return max(self.total) if self.rows else 0

    def slot_map(self) -> SlotMap:
        """The reference's write/read slot tensors for this append, computed
        from the device block tables (cache/kv.py:88-99)."""
        c = self.cache
        offsets, off = [], 0
        for n in self.n_new:
            offsets.append(off)
            off += n
        write, write_index, read = ops.slot_map(c._store.tensor, self.meta, self.batch, c.block_size, self.width,
                                                self.max_total, torch.tensor(offsets, dtype=torch.int32,
                                                                             device=c.device), off)
        past = torch.tensor(self.past, dtype=torch.long, device=c.device)
        total = torch.tensor(self.total, dtype=torch.long, device=c.device)
        return SlotMap(write, write_index, read, past, total)


class KVCache:
    """Paged K/V for independent sequences (cache/kv.py:18-127)."""

    def __init__(self, n_layers: int, n_kv_heads: int, head_dim: int, num_blocks: int, block_size: int,
                 dtype: torch.dtype, device, max_seqs: int = 64) -> None:
        self.block_size = block_size
        self.device = _gpu_device(device)
        self.n_layers, self.n_kv_heads, self.head_dim = n_layers, n_kv_heads, head_dim
        self.allocator = BlockAllocator(num_blocks, self.device)
        self.k = torch.zeros(n_layers, num_blocks, n_kv_heads, block_size, head_dim, dtype=dtype, device=self.device)
        self.v = torch.zeros(n_layers, num_blocks, n_kv_heads, head_dim, block_size, dtype=dtype, device=self.device)
        self.tables: dict[int, BlockTable] = {}
        self._store = _TableStore(max_seqs, num_blocks, self.device)
        self.bytes_per_slot = 2 * n_layers * n_kv_heads * head_dim * self.k.element_size()
        self.graphs: dict = {}  # captured forwards over this cache (lm/graphs.py)

    @property
    def dtype(self) -> torch.dtype:
        return self.k.dtype

    @classmethod
    def for_model(cls, config, num_blocks: int, block_size: int, dtype: torch.dtype, device) -> "KVCache":
        head_dim = getattr(config, "head_dim", None) or config.hidden_size // config.num_attention_heads
        return cls(config.num_hidden_layers, config.num_key_value_heads, head_dim, num_blocks, block_size, dtype,
                   device)

    @classmethod
    def contiguous(cls, config, max_batch: int, max_seq_len: int, dtype: torch.dtype, device) -> "KVCache":
        # one max_seq_len block per sequence, on the same code
        return cls.for_model(config, max_batch, max_seq_len, dtype, device)

    # -- sequences -----------------------------------------------------------
    def add(self, seq_id: int) -> None:
        if seq_id in self.tables:
            raise ValueError(f"sequence {seq_id} already present")
        self.tables[seq_id] = BlockTable(store=self._store, row=self._store.take())

    def free(self, seq_id: int) -> None:
        table = self.tables[seq_id]
        table._shrink(0, self.allocator, self.block_size)
        del self.tables[seq_id]
        self._store.give(table.row)

    def length(self, seq_id: int) -> int:
        return self.tables[seq_id].length

    def truncate(self, seq_id: int, length: int) -> None:
        # Blocks wholly past `length` go back to the free list (queued).  Slots
        # past `length` in the kept block are stale but never read: attention
        # stops at each row's total, and the next append overwrites them first.
        self.tables[seq_id]._shrink(length, self.allocator, self.block_size)

    def flush(self) -> None:
        self.allocator.flush()

    # -- append --------------------------------------------------------------
    def append(self, seq_ids: list[int], n_new: list[int]) -> PagedStep:
        """Reserve slots for n_new[b] tokens on each row; lengths advance now.
        Rows grow in order and an OutOfBlocks leaves earlier rows grown, as in
        cache/kv.py:83-85."""
        width = max(n_new)
        past = [self.tables[s].length for s in seq_ids]
        pops: list[tuple[int, int, int]] = []
        alloc = self.allocator
        failure = None
        for seq_id, n in zip(seq_ids, n_new):
            table = self.tables[seq_id]
            needed = table._need(table.length + n, self.block_size)
            if needed > alloc.num_free:
                failure = OutOfBlocks(f"need {needed} blocks, {alloc.num_free} free")
                break
            if needed > 0:
                pops.append((table.row, len(table), needed))
                alloc._take(needed)
                table._n += needed
            table.length += n
        rows = [self.tables[s].row for s in seq_ids]
        host = rows + past + list(n_new)
        meta = alloc._plan(self._store, pops, tail=host)  # one upload for the plan and the metadata
        if failure is not None:
            raise failure
        if meta is None:
            meta = _upload_i32(host, self.device)
        return PagedStep(self, meta.view(3, len(seq_ids)), rows, past, list(n_new), width)

    def append_steps(self, seq_ids: list[int], steps: list[list[int]]) -> tuple[torch.Tensor, list[PagedStep]]:
        """Reserve slots for several consecutive appends at once, as if
        `append(seq_ids, steps[i])` were called for i = 0, 1, ... in order (same
        block ids, same OutOfBlocks point).  One block-plan launch and one
        metadata upload: returns the int32 [len(steps), 3, B] device metadata
        and a host PagedStep per step (whose `meta` is a view into it)."""
        alloc = self.allocator
        pops: list[tuple[int, int, int]] = []
        host: list[int] = []
        infos = []
        failure = None
        rows = [self.tables[s].row for s in seq_ids]
        for n_new in steps:
            past = [self.tables[s].length for s in seq_ids]
            for seq_id, n in zip(seq_ids, n_new):
                table = self.tables[seq_id]
                needed = table._need(table.length + n, self.block_size)
                if needed > alloc.num_free:
                    failure = OutOfBlocks(f"need {needed} blocks, {alloc.num_free} free")
                    break
                if needed > 0:
                    pops.append((table.row, len(table), needed))
                    alloc._take(needed)
                    table._n += needed
                table.length += n
            if failure is not None:
                break
            host += rows + past + list(n_new)
            infos.append((past, list(n_new)))
        metas = alloc._plan(self._store, pops, tail=host)
        if failure is not None:
            raise failure
        if metas is None:
            metas = _upload_i32(host, self.device)
        metas = metas.view(len(steps), 3, len(seq_ids))
        out = [PagedStep(self, metas[i], rows, past, n_new, max(n_new)) for i, (past, n_new) in enumerate(infos)]
        return metas, out

    # -- per-layer data movement ---------------------------------------------
    def write(self, layer: int, step: PagedStep, k: torch.Tensor, v: torch.Tensor) -> None:
        """k, v: [B, H_kv, T, d] for the tokens passed to `append`, right-padded."""
        ops.kv_write(k, v, step.meta, step.batch, step.width, self._store.tensor, self.block_size, self.k[layer],
                     self.v[layer])

    def gather(self, layer: int, step: PagedStep) -> tuple[torch.Tensor, torch.Tensor]:
        """[B, H_kv, S, d] copies of every cached position (zeros past each
        row's total).  For inspection; attention reads the blocks in place."""
        return ops.kv_gather(self.k[layer], self.v[layer], step.meta, step.batch, self._store.tensor,
                             self.block_size, step.max_total)

    @property
    def table_tensor(self) -> torch.Tensor:
        return self._store.tensor

    def stats(self) -> FragmentationStats:
        return FragmentationStats(
            block_size=self.block_size,
            bytes_per_slot=self.bytes_per_slot,
            blocks_in_use=self.allocator.num_used,
            peak_blocks_in_use=self.allocator.peak_used,
            slots_used=sum(t.length for t in self.tables.values()),
        )

