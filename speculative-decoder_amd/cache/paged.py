"""Paged block allocation with device-resident block ids.

Same API and the same block ids as the reference (cache/paged.py:7-105): a
LIFO free list that hands out 0, 1, 2, ... first and returns the most
recently freed block next; tables that grow to ceil(length / block_size)
blocks and shrink by freeing their tail in table order.

What changes is where the ids live.  The free stack, the "used" marks and the
table rows are int32 tensors on the GPU, and every move of ids between them
is one launch of the block-plan kernel (pushes for rollback/release, then
pops for growth).  The host only keeps counts (free blocks, blocks per
table, lengths), which are enough to raise OutOfBlocks before anything
changes, exactly where the reference raises it.  Ids reach the host only
when asked for (`BlockTable.blocks`, `BlockAllocator.allocate`, `check`).
"""
from __future__ import annotations

import math
from dataclasses import dataclass

import torch

from specdec import ops


class OutOfBlocks(RuntimeError):
    """cache/paged.py:7-8"""


def _gpu_device(device) -> torch.device:
    if device is None:
        if not torch.cuda.is_available():
            raise RuntimeError("paged blocks live in GPU memory and no GPU is visible")
        return torch.device("cuda", torch.cuda.current_device())
    dev = torch.device(device)
    if dev.type != "cuda":
        raise RuntimeError(f"paged blocks live in GPU memory; got device {dev}")
    if dev.index is None:
        dev = torch.device("cuda", torch.cuda.current_device())
    return dev


def _upload_i32(values: list[int], device: torch.device) -> torch.Tensor:
    """An int32 device copy of `values` (a few hundred bytes: from pageable
    memory, which costs the host less here than pinning a fresh buffer)."""
    return torch.tensor(values, dtype=torch.int32).to(device, non_blocking=True)


class _TableStore:
    """int32 [rows, cap] block-table rows on the GPU plus a host free list of rows."""

    def __init__(self, rows: int, cap: int, device: torch.device) -> None:
        self.device = device
        self.tensor = torch.zeros(max(rows, 1), max(cap, 1), dtype=torch.int32, device=device)
        self._free_rows = list(range(self.tensor.shape[0] - 1, -1, -1))

    def take(self) -> int:
        if not self._free_rows:
            old = self.tensor
            grown = torch.zeros(2 * old.shape[0], old.shape[1], dtype=torch.int32, device=self.device)
            grown[: old.shape[0]].copy_(old)
            self.tensor = grown
            self._free_rows = list(range(grown.shape[0] - 1, old.shape[0] - 1, -1))
        return self._free_rows.pop()

    def give(self, row: int) -> None:
        self._free_rows.append(row)

    def ensure_cap(self, cap: int) -> None:
        if cap > self.tensor.shape[1]:
            old = self.tensor
            grown = torch.zeros(old.shape[0], max(cap, 2 * old.shape[1]), dtype=torch.int32, device=self.device)
            grown[:, : old.shape[1]].copy_(old)
            self.tensor = grown


class BlockAllocator:
    """cache/paged.py:11-46 with the free list on the GPU.

    `num_free`, `num_used` and `peak_used` are host counts kept in step with
    every operation.  Pushes of a KVCache's rollbacks may be queued and are
    applied, in order, before the next device operation on this allocator."""

    def __init__(self, num_blocks: int, device=None) -> None:
        self.num_blocks = num_blocks
        self.device = _gpu_device(device)
        # stack[i] = N-1-i: the top of the stack (last index) is block 0
        self._stack = torch.arange(num_blocks - 1, -1, -1, dtype=torch.int32, device=self.device)
        self._used = torch.zeros(max(num_blocks, 1), dtype=torch.uint8, device=self.device)
        self._free = num_blocks  # logical free count, pending pushes included
        self._dev_top = num_blocks  # stack top as of the last applied plan
        self._pending: list[tuple[_TableStore, int, int, int]] = []  # (store, row, col, count) pushes
        self.peak_used = 0
        self._one = _TableStore(1, 1, self.device)

    @property
    def num_free(self) -> int:
        return self._free

    @property
    def num_used(self) -> int:
        return self.num_blocks - self._free

    # -- device plan ---------------------------------------------------------
    def _plan(self, store: _TableStore | None, pops: list[tuple[int, int, int]], popped=None,
              tail: list[int] | None = None) -> torch.Tensor | None:
        """Apply every queued push (grouped per store, in order) and then `pops`
        (row, col, count) on `store`, in one launch per store.  `tail` (int32
        values the caller needs on the device, e.g. a forward's row metadata)
        rides in the last launch's upload; its device copy is returned, or
        None when nothing was launched."""
        tail_dev = None
        groups: list[tuple[_TableStore, list[tuple[int, int, int]]]] = []
        for st, row, col, cnt in self._pending:
            if groups and groups[-1][0] is st:
                groups[-1][1].append((row, col, cnt))
            else:
                groups.append((st, [(row, col, cnt)]))
        self._pending = []
        if pops and (not groups or groups[-1][0] is not store):
            groups.append((store, []))
        for i, (st, pushes) in enumerate(groups):
            last = i == len(groups) - 1
            these_pops = pops if last else []
            entries: list[int] = []
            off = 0
            for row, col, cnt in pushes:
                entries += [row, col, cnt, off]
                off += cnt
            pushed = off
            off = 0
            for row, col, cnt in these_pops:
                entries += [row, col, cnt, off]
                off += cnt
            if not entries:
                continue
            if last and tail is not None:
                both = _upload_i32(entries + tail, self.device)
                up, tail_dev = both[: len(entries)], both[len(entries):]
            else:
                up = _upload_i32(entries, self.device)
            ops.block_plan(st.tensor, self._stack, self._used, self._dev_top, up, len(pushes), len(these_pops),
                           popped if last else None)
            self._dev_top += pushed - off
        return tail_dev

    def _queue_push(self, store: _TableStore, row: int, col: int, count: int) -> None:
        if count > 0:
            self._pending.append((store, row, col, count))
            self._free += count

    def _take(self, count: int) -> None:
        self._free -= count
        self.peak_used = max(self.peak_used, self.num_used)

    def flush(self) -> None:
        if self._pending:
            self._plan(None, [])

    # -- reference API -------------------------------------------------------
    def allocate(self) -> int:
        if self._free == 0:
            raise OutOfBlocks(f"all {self.num_blocks} blocks in use")
        self._take(1)
        self._plan(self._one, [(0, 0, 1)])
        return int(self._one.tensor[0, 0].item())

    def free(self, block: int) -> None:
        err = ValueError(f"block {block} is not allocated (double free or foreign id)")
        if not (0 <= block < self.num_blocks) or self._free >= self.num_blocks:
            raise err
        self.flush()
        status = torch.empty(1, dtype=torch.int32, device=self.device)
        ops.block_free_checked(self._stack, self._used, self._dev_top, block, status)
        if int(status.item()):
            raise err
        self._dev_top += 1
        self._free += 1

    def check(self) -> None:
        self.flush()
        stack = self._stack[: self._dev_top].cpu().tolist()
        used = set(torch.nonzero(self._used[: self.num_blocks].cpu()).flatten().tolist())
        free = set(stack)
        assert self._dev_top == self._free, "host and device free counts disagree"
        assert len(free) == len(stack), "duplicate id in free list"
        assert not (free & used), "block both free and used"
        assert free | used == set(range(self.num_blocks)), "block leaked"


class BlockTable:
    """cache/paged.py:49-76.  `length` and the block count are host ints; the
    block ids are one row of a device table store.

    `BlockTable(blocks=[7, 2], length=6)` builds a standalone table as in the
    reference; a KVCache hands out rows of its shared store instead."""

    def __init__(self, blocks: list[int] | None = None, length: int = 0, *, store: _TableStore | None = None,
                 row: int | None = None, device=None) -> None:
        blocks = list(blocks or [])
        if store is None:
            store = _TableStore(1, max(len(blocks), 1), _gpu_device(device))
            row = store.take()
        self._store = store
        self._row = row
        self.length = length
        self._n = len(blocks)
        if blocks:
            store.ensure_cap(len(blocks))
            store.tensor[row, : len(blocks)] = torch.tensor(blocks, dtype=torch.int32)

    @property
    def blocks(self) -> list[int]:
        return self._store.tensor[self._row, : self._n].cpu().tolist()

    @property
    def row(self) -> int:
        return self._row

    def __len__(self) -> int:
        return self._n

    def _need(self, length: int, block_size: int) -> int:
        return math.ceil(length / block_size) - self._n

    def grow_to(self, length: int, allocator: BlockAllocator, block_size: int) -> None:
        needed = self._need(length, block_size)
        # checked before anything moves, so a failed grow leaves both untouched
        if needed > allocator.num_free:
            raise OutOfBlocks(f"need {needed} blocks, {allocator.num_free} free")
        if needed > 0:
            self._store.ensure_cap(self._n + needed)
            allocator._take(needed)
            allocator._plan(self._store, [(self._row, self._n, needed)])
            self._n += needed
        self.length = length

    def _shrink(self, length: int, allocator: BlockAllocator, block_size: int) -> None:
        if length > self.length:
            raise ValueError(f"cannot shrink length {self.length} to {length}")
        keep = math.ceil(length / block_size)
        if self._n > keep:
            allocator._queue_push(self._store, self._row, keep, self._n - keep)
            self._n = keep
        self.length = length

    def shrink_to(self, length: int, allocator: BlockAllocator, block_size: int) -> None:
        self._shrink(length, allocator, block_size)
        allocator.flush()

    def slots(self, start: int, stop: int, block_size: int) -> torch.Tensor:
        if start < 0 or (stop > start and math.ceil(stop / block_size) > self._n):
            raise IndexError(f"positions [{start}, {stop}) exceed the table's {self._n} blocks")
        return ops.block_slots(self._store.tensor[self._row], start, stop, block_size)


@dataclass(frozen=True)
class FragmentationStats:
    """cache/paged.py:79-105"""

    block_size: int
    bytes_per_slot: int
    blocks_in_use: int
    peak_blocks_in_use: int
    slots_used: int

    @property
    def slots_allocated(self) -> int:
        return self.blocks_in_use * self.block_size

    @property
    def waste(self) -> float:
        # the unused tail of each sequence's last block; fixed-size blocks have
        # no external fragmentation
        if self.slots_allocated == 0:
            return 0.0
        return 1.0 - self.slots_used / self.slots_allocated

    @property
    def bytes_in_use(self) -> int:
        return self.slots_allocated * self.bytes_per_slot

    @property
    def peak_bytes(self) -> int:
        return self.peak_blocks_in_use * self.block_size * self.bytes_per_slot
