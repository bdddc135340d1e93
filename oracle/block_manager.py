"""CPU restatement of the reference's paged block manager (test oracle).

Test infrastructure only: imported by tests/, never by the product.

Restates runtime/src/cache/block.rs:78-352 (BlockManager, the state
behind PyBlockManager, runtime/src/lib.rs:82-168) with plain Python lists:
the free list is a stack initialised to [0, 1, ..., n-1], allocation pops
from its end, release pushes to its end; reference counts saturate at 0;
free_block pushes a block whose count reaches 0 even if it is already on
the free list (block.rs:199-210); assign_cached_blocks does not take blocks
off the free list (block.rs:214-231).

Adds the copy-on-write rule of this build's prepare_writes (the reference
has none): per write in order, grow the table to cover the write, then
replace each touched block whose count is above 1, lowest position first,
by a fresh block, recording (old, new).
"""

from __future__ import annotations


class OutOfBlocks(RuntimeError):
    pass


class BlockManagerRef:
    def __init__(self, num_blocks: int, block_size: int) -> None:
        if num_blocks <= 0 or block_size <= 0:
            raise ValueError("num_blocks and block_size must be positive")
        self.num_blocks = num_blocks
        self.block_size = block_size
        self.rc = [0] * num_blocks
        self.free_list = list(range(num_blocks))
        self.tables: dict[str, list[int]] = {}
        self.lens: dict[str, int] = {}

    def _ceil(self, tokens: int) -> int:
        return -(-tokens // self.block_size)

    def _pop(self) -> int:
        b = self.free_list.pop()
        self.rc[b] += 1
        return b

    def allocate(self, rid: str, num_tokens: int) -> list[int]:
        if rid in self.tables:
            raise OutOfBlocks("duplicate request id")
        need = self._ceil(num_tokens)
        if need > len(self.free_list):
            raise OutOfBlocks(f"need {need}")
        self.tables[rid] = [self._pop() for _ in range(need)]
        return list(self.tables[rid])

    def free(self, rid: str) -> None:
        table = self.tables.pop(rid, None)
        if table is None:
            return
        for b in table:
            self.rc[b] = max(self.rc[b] - 1, 0)
            if self.rc[b] == 0:
                self.free_list.append(b)
        self.lens.pop(rid, None)

    def free_block(self, b: int) -> None:
        if not 0 <= b < self.num_blocks:
            return
        self.rc[b] = max(self.rc[b] - 1, 0)
        if self.rc[b] == 0:
            self.free_list.append(b)

    def increment_ref_count(self, b: int) -> None:
        if 0 <= b < self.num_blocks:
            self.rc[b] += 1

    def assign_cached_blocks(self, rid: str, ids: list[int]) -> None:
        for b in ids:
            if 0 <= b < self.num_blocks:
                self.rc[b] += 1
        self.tables[rid] = list(ids) + self.tables.get(rid, [])

    def ensure_blocks(self, rid: str, target_tokens: int) -> None:
        have = len(self.tables.get(rid, [])) * self.block_size
        if have >= target_tokens:
            return
        extra = self._ceil(target_tokens - have)
        if extra > len(self.free_list):
            raise OutOfBlocks(f"need {extra}")
        t = self.tables.setdefault(rid, [])
        t.extend(self._pop() for _ in range(extra))

    def share_prefix(self, src: str, dst: str, prefix_len: int) -> list[int]:
        if src not in self.tables:
            raise ValueError("source not found")
        if dst in self.tables:
            raise ValueError("destination exists")
        n = self._ceil(prefix_len)
        if n > len(self.tables[src]):
            raise ValueError("prefix longer than source")
        shared = self.tables[src][:n]
        for b in shared:
            self.rc[b] += 1
        self.tables[dst] = list(shared)
        return list(shared)

    def get_blocks(self, rid: str) -> list[int]:
        if rid not in self.tables:
            raise KeyError(rid)
        return list(self.tables[rid])

    def num_free_blocks(self) -> int:
        return len(self.free_list)

    def prepare_writes(self, writes: list[tuple[str, int, int]]) -> tuple[list[int], list[tuple[int, int]]]:
        bs = self.block_size
        need = 0
        for rid, start, count in writes:
            if count == 0:
                continue
            t = self.tables.get(rid, [])
            want = self._ceil(start + count)
            need += max(want - len(t), 0)
            need += sum(1 for j in range(start // bs, min(want, len(t))) if self.rc[t[j]] > 1)
        if need > len(self.free_list):
            raise OutOfBlocks(f"need {need}")
        slots: list[int] = []
        copies: list[tuple[int, int]] = []
        for rid, start, count in writes:
            if count == 0:
                continue
            t = self.tables.setdefault(rid, [])
            want = self._ceil(start + count)
            have = len(t)
            while len(t) < want:
                t.append(self._pop())
            for j in range(start // bs, min(have, want)):
                old = t[j]
                if self.rc[old] > 1:
                    new = self._pop()
                    self.rc[old] -= 1
                    t[j] = new
                    copies.append((old, new))
            slots += [t[p // bs] * bs + p % bs for p in range(start, start + count)]
            self.lens[rid] = max(self.lens.get(rid, 0), start + count)
        return slots, copies
