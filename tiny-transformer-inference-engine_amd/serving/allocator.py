"""Physical KV block allocator — drop-in for serving/allocator.py.

Observable contract (reference: serving/allocator.py:1-43,
tests/test_block_allocator.py): block 0 is never handed out, so a
zero-padded block table cannot alias a live block; blocks that were never
used come out in increasing id order (1, 2, 3, ...); freed blocks are handed
out again before any unused one, most recently freed first; a failed `free`
raises ValueError and changes nothing; running out raises RuntimeError.
Block tables built on top of it are compared bit for bit, so this order is
part of the interface.

Representation: a high-water mark (the lowest id never handed out), a stack
of returned ids, and one in-use byte per block.
"""
from __future__ import annotations


class BlockAllocator:
    """Physical KV block ids for one pool; id 0 stays reserved."""

    def __init__(self, num_blocks: int):
        assert num_blocks >= 2, "need block 0 plus at least one usable block"
        self.num_blocks = num_blocks
        self._high = 1                 # ids >= _high have never been handed out
        self._returned: list[int] = []  # top of the stack = most recently freed
        self._in_use = bytearray(num_blocks)

    @property
    def num_free(self) -> int:
        return (self.num_blocks - self._high) + len(self._returned)

    @property
    def num_usable(self) -> int:
        return self.num_blocks - 1

    def can_allocate(self, n: int) -> bool:
        return n <= self.num_free

    def allocate(self) -> int:
        if self._returned:
            b = self._returned.pop()
        elif self._high < self.num_blocks:
            b = self._high
            self._high += 1
        else:
            raise RuntimeError("out of KV blocks")
        self._in_use[b] = 1
        return b

    def allocate_n(self, n: int) -> list[int]:
        if not self.can_allocate(n):
            raise RuntimeError(f"need {n} blocks, only {self.num_free} free")
        return [self.allocate() for _ in range(n)]

    def free(self, blocks: list[int]) -> None:
        """Return `blocks` (in order) to the allocator. Each id is released
        tentatively; the first bad one (outside [1, num_blocks), not in use,
        or listed twice) rolls the earlier ones back and raises ValueError,
        so a failed call leaves the allocator as it was."""
        done = 0
        try:
            for b in blocks:
                if not (0 < b < self.num_blocks):
                    raise ValueError(f"invalid block id {b}")
                if not self._in_use[b]:
                    raise ValueError(f"double free of block {b}")
                self._in_use[b] = 0
                done += 1
        except ValueError:
            for b in blocks[:done]:
                self._in_use[b] = 1
            raise
        self._returned.extend(blocks)
