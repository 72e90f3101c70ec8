"""CPU model of the paged-KV bookkeeping the device page table reproduces. TEST INFRASTRUCTURE ONLY.

Restates, over plain integer lists, the reference's BlockAllocator (src/state.py:78-103: a free list whose pop()
returns block 0 first; freed blocks appended in reverse, so they come back in table order), PagedSequence growth
(src/state.py:148-157: the blocks a sequence is missing for positions < end, taken all or nothing) and the 0-padded
tables of batch_layout (src/state.py:124-128), for a batch advanced in order. One difference is deliberate and
matches the device version: a batch whose total need exceeds the free blocks takes nothing for any sequence (the
reference's per-sequence loop would have let the sequences before the failing one keep their new blocks).
"""


class PagesModel:
    def __init__(self, num_blocks: int, max_seqs: int, max_blocks: int, block_size: int):
        self.num_blocks, self.max_seqs, self.max_blocks, self.bs = num_blocks, max_seqs, max_blocks, block_size
        self.free = list(range(num_blocks - 1, -1, -1))          # the end of the list is handed out next
        self.tables = [[] for _ in range(max_seqs)]
        self.lens = [0] * max_seqs
        self.status = 0

    def _blocks(self, n: int) -> int:
        return -(-n // self.bs)

    def advance(self, rows: list[int], n_new: int):
        """-> (slots, lens after) or None when the step fails (status set, nothing changed)."""
        if any(r < 0 or r >= self.max_seqs for r in rows):
            self.status = 4
            return None
        if len(set(rows)) != len(rows):                          # one sequence grown twice in a step
            self.status = 5
            return None
        needs = [self._blocks(self.lens[r] + n_new) - self._blocks(self.lens[r]) for r in rows]
        if any(self._blocks(self.lens[r] + n_new) > self.max_blocks for r in rows):
            self.status = 2
            return None
        if sum(needs) > len(self.free):
            self.status = 1
            return None
        slots, lens = [], []
        for r, need in zip(rows, needs):
            for _ in range(need):
                self.tables[r].append(self.free.pop())
            for p in range(self.lens[r], self.lens[r] + n_new):
                slots.append(self.tables[r][p // self.bs] * self.bs + p % self.bs)
            self.lens[r] += n_new
            lens.append(self.lens[r])
        return slots, lens

    def release(self, rows: list[int]) -> None:
        if any(r < 0 or r >= self.max_seqs for r in rows):
            self.status = 4
            return
        if len(set(rows)) != len(rows):                          # a double free (BlockAllocator.free refuses it)
            self.status = 5
            return
        for r in rows:
            self.free.extend(reversed(self.tables[r]))
            self.tables[r] = []
            self.lens[r] = 0

    def table_rows(self, rows: list[int], width: int) -> list[list[int]]:
        return [(self.tables[r] + [0] * width)[:width] for r in rows]
