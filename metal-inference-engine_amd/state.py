"""Per-sequence decode state with the reference engine's layouts (src/state.py), for pools that live on a ROCm GPU.

Layouts kept exactly, because the HIP kernels index them in place:
  * paged KV pool    k, v: [n_layers, num_blocks, block_size, n_kv_heads, head_dim], the two halves of one zeroed
                      [2, ...] buffer (src/state.py:11-17, 106-114);
  * block tables     int32 [B, max_nb], rows padded with 0; lens int32 [B] (src/state.py:119-129);
  * DeltaNet slots   S: [max_seqs, n_linear, H, dk, dv] fp32, conv: [max_seqs, n_linear, K-1, C] fp32
                      (src/state.py:420-429); a slot is zeroed when released (src/state.py:467-470);
  * grouped pool     k, v: [G, units, block_size, n_kv_heads, head_dim] for layer groups with sliding-window rings
                      (src/state.py:195-359); one group slot is a paged layer as above.
Allocation is host-side bookkeeping (free list, all-or-nothing growth). KV scatter and gather run as HIP kernels
when the pool is on a GPU (librk_path.so: rk_kv_write / rk_kv_gather) and as torch indexing on the CPU.
"""
import math

import torch


def kv_buffers(shape: tuple, device, dtype) -> tuple[torch.Tensor, torch.Tensor]:
    """K and V as contiguous halves of one zero-filled [2, *shape] allocation (src/state.py:11-17)."""
    both = torch.zeros(2, *shape, device=device, dtype=dtype)
    return both[0], both[1]


def to_device(t: torch.Tensor, device) -> torch.Tensor:
    """A small host tensor (ids, positions, tables) copied to `device` (src/state.py:20-29). On a ROCm device the
    copy comes from a private pinned clone and does not wait for queued kernels; the clone keeps the host bytes
    unchanged until the copy has read them, whatever the caller does with its own tensor afterwards."""
    dev = torch.device(device)
    if dev.type != "cuda":
        return t.to(dev)
    return t.clone().pin_memory().to(dev, non_blocking=True)


def _slots(blocks: torch.Tensor, offsets: torch.Tensor, block_size: int) -> torch.Tensor:
    return blocks.to(torch.int64) * block_size + offsets.to(torch.int64)


class ContiguousKVCache:
    """Standalone (unpooled) cache, one buffer per layer: k/v [n_layers, max_len, Hkv, d] (src/state.py:32-71)."""

    def __init__(self, n_layers: int, n_kv_heads: int, head_dim: int, max_len: int, device="cpu",
                 dtype: torch.dtype = torch.float32):
        self.max_len = max_len
        self.k, self.v = kv_buffers((n_layers, max_len, n_kv_heads, head_dim), device, dtype)
        self.length = 0

    def _check(self, end: int) -> None:
        if end > self.max_len:
            raise ValueError(f"KV cache full: need {end} positions, capacity {self.max_len}")

    def write(self, layer: int, start: int, k: torch.Tensor, v: torch.Tensor) -> None:
        end = start + k.shape[0]
        self._check(end)
        self.k[layer, start:end] = k.to(self.k.dtype)
        self.v[layer, start:end] = v.to(self.v.dtype)

    def read(self, layer: int, end: int, lo: int = 0) -> tuple[torch.Tensor, torch.Tensor]:
        return self.k[layer, lo:end], self.v[layer, lo:end]

    def advance(self, n: int) -> None:
        self.length += n

    def reserve(self, end: int) -> None:
        self._check(end)

    def bytes_used(self) -> int:
        return 2 * self.k[:, : self.length].numel() * self.k.element_size()

    def fork(self) -> "ContiguousKVCache":
        L, max_len, h, d = self.k.shape
        twin = ContiguousKVCache(L, h, d, max_len, device=self.k.device, dtype=self.k.dtype)
        n = self.length
        twin.k[:, :n] = self.k[:, :n]
        twin.v[:, :n] = self.v[:, :n]
        twin.length = n
        return twin


class OutOfBlocks(RuntimeError):
    """No free KV block (or state slot) is left in the shared pool."""


class BlockAllocator:
    """Free-list allocator of fixed-size KV blocks (src/state.py:78-103). Blocks come out in ascending order from a
    fresh pool (block 0 first); a double free or a free of a block never handed out raises ValueError."""

    def __init__(self, num_blocks: int):
        self.num_blocks = num_blocks
        self.free_list = list(reversed(range(num_blocks)))   # the end of the list is handed out next
        self.in_use: set[int] = set()

    @property
    def num_free(self) -> int:
        return len(self.free_list)

    def allocate(self) -> int:
        if not self.free_list:
            raise OutOfBlocks(f"all {self.num_blocks} KV blocks are in use")
        blk = self.free_list.pop()
        self.in_use.add(blk)
        return blk

    def free(self, blocks: list[int]) -> None:
        unknown = sorted({b for b in blocks if b not in self.in_use})
        if unknown or len(set(blocks)) != len(blocks):
            raise ValueError(f"freeing KV blocks that are not in use (or twice): {unknown[:8]}")
        self.in_use.difference_update(blocks)
        self.free_list.extend(blocks[::-1])


class PagedKVPool:
    """Blocks of KV shared by all sequences: k/v [n_layers, num_blocks, block_size, Hkv, d] (src/state.py:106-134)."""

    def __init__(self, n_layers: int, n_kv_heads: int, head_dim: int, num_blocks: int, block_size: int = 16,
                 device="cpu", dtype: torch.dtype = torch.float32):
        self.block_size = block_size
        self.k, self.v = kv_buffers((n_layers, num_blocks, block_size, n_kv_heads, head_dim), device, dtype)
        self.allocator = BlockAllocator(num_blocks)
        self.unit_bytes = 2 * self.k[:, 0].numel() * self.k.element_size()

    def new_sequence(self) -> "PagedSequence":
        return PagedSequence(self)

    def batch_layout(self, seqs: list["PagedSequence"], starts: list[int]):
        """One decode step: the (block, offset) each new token is written to, and every sequence's block table
        (0-padded to the widest) and length after it, as device tensors (blocks, offsets: int64; tables, lens:
        int32), built once per step and shared by all layers."""
        bs, dev = self.block_size, self.k.device
        width = max(len(s.block_table) for s in seqs)
        blocks = torch.tensor([s.block_table[p // bs] for s, p in zip(seqs, starts)], dtype=torch.int64)
        offsets = torch.tensor([p % bs for p in starts], dtype=torch.int64)
        tables = torch.tensor([s.block_table + [0] * (width - len(s.block_table)) for s in seqs], dtype=torch.int32)
        lens = torch.tensor([p + 1 for p in starts], dtype=torch.int32)
        return tuple(to_device(t, dev) for t in (blocks, offsets, tables, lens))

    def prefill_layout(self, seqs: list["PagedSequence"], starts: list[int], lengths: list[int]):
        """Packed prefill of len(seqs) segments, segment s adding lengths[s] tokens at positions starts[s] .. of
        seqs[s] (blocks already reserved): (tables [S, max_nb] int32 on the pool's device, cu_seqlens, starts) with
        cu_seqlens the S + 1 row offsets of the packed batch (the layout src/models/packing.py:21-31 packs)."""
        width = max(1, max(len(s.block_table) for s in seqs))
        tables = torch.tensor([s.block_table + [0] * (width - len(s.block_table)) for s in seqs], dtype=torch.int32)
        cu = [0]
        for n in lengths:
            cu.append(cu[-1] + n)
        return to_device(tables, self.k.device), cu, list(starts)

    def write_rows(self, layer: int, slots: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> None:
        """k, v [n, Hkv, d] into flat row indices slots = block * block_size + offset of one layer."""
        if self.k.is_cuda:
            from native.kernels import kv_write
            kv_write(self.k[layer], self.v[layer], slots, k, v)
        else:
            kl = self.k[layer].view(-1, *self.k.shape[3:])
            vl = self.v[layer].view(-1, *self.v.shape[3:])
            kl[slots.long()] = k.to(self.k.dtype)
            vl[slots.long()] = v.to(self.v.dtype)

    def write_batch(self, layer: int, blocks: torch.Tensor, offsets: torch.Tensor, k: torch.Tensor, v: torch.Tensor):
        """k, v [B, Hkv, d]: one new token per sequence (src/state.py:131-134)."""
        self.write_rows(layer, _slots(blocks, offsets, self.block_size), k, v)


class PagedSequence:
    """One sequence's block table into a PagedKVPool (src/state.py:137-193); same interface as ContiguousKVCache."""

    def __init__(self, pool: PagedKVPool):
        self.pool = pool
        self.block_table: list[int] = []
        self.length = 0

    def _ensure(self, end: int) -> None:
        """Grow the table to cover positions < end, all or nothing: if the pool cannot supply every missing block,
        raise OutOfBlocks before taking any."""
        missing = math.ceil(end / self.pool.block_size) - len(self.block_table)
        if missing <= 0:
            return
        free = self.pool.allocator.num_free
        if missing > free:
            raise OutOfBlocks(f"need {missing} more KV blocks, only {free} free")
        self.block_table += [self.pool.allocator.allocate() for _ in range(missing)]

    def reserve(self, end: int) -> None:
        self._ensure(end)

    def write(self, layer: int, start: int, k: torch.Tensor, v: torch.Tensor) -> None:
        end = start + k.shape[0]
        self._ensure(end)
        bs = self.pool.block_size
        pos = torch.arange(start, end, dtype=torch.int64)
        table = torch.tensor(self.block_table, dtype=torch.int64)
        slots = table[pos // bs] * bs + pos % bs
        self.pool.write_rows(layer, to_device(slots, self.pool.k.device), k, v)

    def read(self, layer: int, end: int, lo: int = 0) -> tuple[torch.Tensor, torch.Tensor]:
        """Positions lo .. end-1 gathered into contiguous [end - lo, Hkv, d]; only their blocks are touched."""
        bs = self.pool.block_size
        first, last = lo // bs, math.ceil(end / bs)
        if self.pool.k.is_cuda:
            from native.kernels import kv_gather
            table = to_device(torch.tensor(self.block_table[:last], dtype=torch.int32), self.pool.k.device)
            return kv_gather(self.pool.k[layer], self.pool.v[layer], table, lo, end)
        idx = torch.tensor(self.block_table[first:last], dtype=torch.int64)
        rows = slice(lo - first * bs, end - first * bs)
        return self.pool.k[layer, idx].flatten(0, 1)[rows], self.pool.v[layer, idx].flatten(0, 1)[rows]

    def advance(self, n: int) -> None:
        self.length += n

    def free(self) -> None:
        self.pool.allocator.free(self.block_table)
        self.block_table = []
        self.length = 0

    def bytes_used(self) -> int:
        p = self.pool
        return 2 * len(self.block_table) * p.k[0, 0].numel() * p.k.shape[0] * p.k.element_size()


def _write_layer(k_layer: torch.Tensor, v_layer: torch.Tensor, slots: torch.Tensor, k: torch.Tensor,
                 v: torch.Tensor) -> None:
    """k, v [n, Hkv, d] into rows slots = unit * block_size + offset of one pool layer [units, bs, Hkv, d]: the HIP
    scatter on a GPU, torch indexing on the CPU."""
    if k_layer.is_cuda:
        from native.kernels import kv_write
        kv_write(k_layer, v_layer, slots, k, v)
    else:
        k_layer.view(-1, *k_layer.shape[2:])[slots.long()] = k.to(k_layer.dtype)
        v_layer.view(-1, *v_layer.shape[2:])[slots.long()] = v.to(v_layer.dtype)


class GroupedKVPool:
    """Paged KV for a model whose layers look back different distances (src/state.py:195-262; Tiny Aya: 9 full and
    27 sliding-window layers), so the sliding layers' memory stops growing past the window.

    Layers are grouped G = gcd(#full, #sliding) at a time (full groups first, then sliding groups); the pool's unit
    is one block of one group's G layers, k / v [G, units, block_size, Hkv, d], and one allocator hands units to all
    groups (units = num_blocks x groups, so num_blocks still counts blocks of every layer). Per sequence a full group
    holds one unit per block; a sliding group a ring of R = ceil((W + max_chunk + bs - 2) / bs) units with logical
    block b in slot b % R, enough for every block one forward of at most max_chunk tokens reads or writes. A layer of
    the pool, k[slot] [units, bs, Hkv, d], has the paged layout the decode kernel reads, through the group's table
    (by absolute block; entries before a sliding window are pad_block and never read). poison=True (tests): a ring
    slot taking a new block is first filled with NaN, so a stale read shows."""

    def __init__(self, layer_windows: list, n_kv_heads: int, head_dim: int, num_blocks: int, block_size: int = 16,
                 max_chunk: int = 512, device="cpu", dtype: torch.dtype = torch.float32, poison: bool = False):
        full = [i for i, w in enumerate(layer_windows) if w is None]
        sliding = [i for i, w in enumerate(layer_windows) if w is not None]
        windows = sorted({w for w in layer_windows if w is not None})
        if len(windows) > 1:
            raise ValueError(f"one sliding window size per model, not {windows}")
        self.window = windows[0] if windows else None
        G = math.gcd(len(full), len(sliding))
        self.groups = [full[i:i + G] for i in range(0, len(full), G)] + \
            [sliding[i:i + G] for i in range(0, len(sliding), G)]
        self.sliding = [False] * (len(full) // G) + [True] * (len(sliding) // G)
        self.layer_map = {layer: (g, j) for g, members in enumerate(self.groups) for j, layer in enumerate(members)}
        self.n_groups, self.block_size, self.poison = len(self.groups), block_size, poison
        self.ring = math.ceil((self.window + max_chunk + block_size - 2) / block_size) if self.window else None
        self.k, self.v = kv_buffers((G, num_blocks * self.n_groups, block_size, n_kv_heads, head_dim), device, dtype)
        self.allocator = BlockAllocator(num_blocks * self.n_groups)
        self.unit_bytes = 2 * self.k[:, 0].numel() * self.k.element_size()
        self.max_step_units = self.n_groups          # a decode step adds at most one unit per group
        self.pad_block = 0

    def blocks_for(self, n: int) -> int:
        """Units a sequence of n positions holds: one per block in a full group, at most R in a sliding one."""
        nb = math.ceil(n / self.block_size)
        return sum(min(self.ring, nb) if sl else nb for sl in self.sliding)

    def new_sequence(self) -> "WindowedSequence":
        return WindowedSequence(self)

    def batch_layout(self, seqs: list["WindowedSequence"], starts: list[int]):
        """One decode step (a new token per sequence at starts[i], units reserved), as device tensors: per group the
        unit each new token goes to (blocks [groups, B] int64, ring slots retagged), offsets [B] int64, per group
        every sequence's table by absolute block (tables [groups, B, max_nb] int32, 0-padded; a sliding group's
        entries before the window are pad_block), lens [B] int32 = starts + 1."""
        bs, W = self.block_size, self.window
        width = max(math.ceil((p + 1) / bs) for p in starts)
        blocks = [[s.unit(g, p // bs, write=True) for s, p in zip(seqs, starts)] for g in range(self.n_groups)]
        tables = []
        for g, sl in enumerate(self.sliding):
            rows = []
            for s, p in zip(seqs, starts):
                first = max(0, p + 1 - W) // bs if sl else 0
                row = [self.pad_block] * first + [s.unit(g, b) for b in range(first, math.ceil((p + 1) / bs))]
                rows.append(row + [self.pad_block] * (width - len(row)))
            tables.append(rows)
        out = (torch.tensor(blocks, dtype=torch.int64), torch.tensor([p % bs for p in starts], dtype=torch.int64),
               torch.tensor(tables, dtype=torch.int32), torch.tensor([p + 1 for p in starts], dtype=torch.int32))
        return tuple(to_device(t, self.k.device) for t in out)

    def write_batch(self, slot: int, blocks: torch.Tensor, offsets: torch.Tensor, k: torch.Tensor, v: torch.Tensor):
        """k, v [B, Hkv, d]: one new token per sequence, for the layer at `slot` of one group (blocks: that group's
        row of batch_layout's blocks)."""
        _write_layer(self.k[slot], self.v[slot], _slots(blocks, offsets, self.block_size), k, v)


class WindowedSequence:
    """One sequence's view of a GroupedKVPool (src/state.py:265-359): a table of units per full group, a ring of
    units per sliding group with the logical block each ring slot holds (its tag). Same interface as PagedSequence;
    block_table is the first group's table."""

    def __init__(self, pool: GroupedKVPool):
        self.pool = pool
        self.tables: list[list[int]] = [[] for _ in range(pool.n_groups)]
        self.tags: list[list[int]] = [[] for _ in range(pool.n_groups)]
        self.length = 0
        self.shared = 0                   # blocks 0 .. shared-1 of every group belong to a borrowed prefix

    @property
    def block_table(self) -> list[int]:
        return self.tables[0]

    def check_forward(self, start: int, end: int) -> None:
        """Refuse, before anything moves, a forward whose blocks (the first query's window .. the last token) do not
        fit in the ring (a chunk longer than the pool's max_chunk)."""
        p = self.pool
        if p.ring is None:
            return
        span = math.ceil(end / p.block_size) - max(0, start - p.window + 1) // p.block_size
        if span > p.ring:
            raise ValueError(f"a forward from position {start} to {end} spans {span} blocks, more than the "
                             f"{p.ring}-block ring (chunks of at most the pool's max_chunk tokens)")

    def reserve(self, end: int) -> None:
        """Take every unit positions < end need, all or nothing (as PagedSequence.reserve)."""
        p = self.pool
        need = p.blocks_for(end) - sum(len(t) for t in self.tables)
        if need <= 0:
            return
        if need > p.allocator.num_free:
            raise OutOfBlocks(f"need {need} more KV units, only {p.allocator.num_free} free")
        nb = math.ceil(end / p.block_size)
        for g, sl in enumerate(p.sliding):
            want = min(p.ring, nb) if sl else nb
            while len(self.tables[g]) < want:
                self.tables[g].append(p.allocator.allocate())
                self.tags[g].append(-1)

    def borrow(self, pin: "WindowedSequence", n: int) -> None:
        """Start this empty sequence from the first n blocks of `pin` (same pool, rings not yet wrapped), shared
        read-only: never written through (unit) or freed (free) by this sequence."""
        p = self.pool
        if self.length or any(self.tables) or pin.pool is not p or n * p.block_size > pin.length or \
                any(sl and pin.tags[g][:n] != list(range(n)) for g, sl in enumerate(p.sliding)):
            raise ValueError("borrow needs an empty sequence and a sequence of the same pool holding blocks 0..n-1")
        self.tables = [t[:n] for t in pin.tables]
        self.tags = [t[:n] for t in pin.tags]
        self.length, self.shared = n * p.block_size, n

    def unit(self, g: int, b: int, write: bool = False) -> int:
        """The unit holding logical block b of group g. Writing to a sliding group's block retags its ring slot
        (poisoning it first when the pool asks); reading a block the ring no longer holds raises."""
        p = self.pool
        i = b % p.ring if p.sliding[g] else b
        if write and i < self.shared:
            raise RuntimeError(f"a write to block {b} of group {g} would overwrite a shared prefix")
        if not p.sliding[g]:
            return self.tables[g][b]
        if self.tags[g][i] != b:
            if not write:
                raise RuntimeError(f"block {b} of group {g} is no longer in the ring (slot {i} holds "
                                   f"{self.tags[g][i]})")
            if p.poison:
                p.k[:, self.tables[g][i]] = float("nan")
                p.v[:, self.tables[g][i]] = float("nan")
            self.tags[g][i] = b
        return self.tables[g][i]

    def write(self, layer: int, start: int, k: torch.Tensor, v: torch.Tensor) -> None:
        end = start + k.shape[0]
        self.reserve(end)
        g, slot = self.pool.layer_map[layer]
        bs = self.pool.block_size
        slots = torch.tensor([self.unit(g, t // bs, write=True) * bs + t % bs for t in range(start, end)],
                             dtype=torch.int64)
        _write_layer(self.pool.k[slot], self.pool.v[slot], to_device(slots, self.pool.k.device), k, v)

    def read(self, layer: int, end: int, lo: int = 0) -> tuple[torch.Tensor, torch.Tensor]:
        """Positions lo .. end-1 of one layer, gathered into contiguous [end - lo, Hkv, d]."""
        g, slot = self.pool.layer_map[layer]
        bs = self.pool.block_size
        b0, nb = lo // bs, math.ceil(end / bs)
        units = [self.unit(g, b) for b in range(b0, nb)]
        kl, vl = self.pool.k[slot], self.pool.v[slot]
        if kl.is_cuda:
            from native.kernels import kv_gather
            table = to_device(torch.tensor([self.pool.pad_block] * b0 + units, dtype=torch.int32), kl.device)
            return kv_gather(kl, vl, table, lo, end)
        idx = torch.tensor(units, dtype=torch.int64)
        rows = slice(lo - b0 * bs, end - b0 * bs)
        return kl[idx].flatten(0, 1)[rows], vl[idx].flatten(0, 1)[rows]

    def advance(self, n: int) -> None:
        self.length += n

    def free(self) -> None:
        self.pool.allocator.free([u for t in self.tables for u in t[self.shared:]])   # a borrowed prefix stays
        self.tables = [[] for _ in range(self.pool.n_groups)]
        self.tags = [[] for _ in range(self.pool.n_groups)]
        self.length = self.shared = 0

    def bytes_used(self) -> int:
        return (sum(len(t) for t in self.tables) - self.shared * len(self.tables)) * self.pool.unit_bytes


class HybridState:
    """A Qwen3.5 sequence: a KV cache for the attention layers plus, for the DeltaNet layers, a fixed-size recurrent
    state S [n_linear, H, dk, dv] and conv tail [n_linear, K-1, C] (src/state.py:362-417). States made by a
    HybridPool are views of one pool slot `seq`."""

    def __init__(self, kv, n_linear: int = 0, n_heads: int = 0, dk: int = 0, dv: int = 0, conv_dim: int = 0,
                 conv_k: int = 1, device="cpu", pool: "HybridPool | None" = None, seq: int | None = None):
        self.kv, self.pool, self.seq = kv, pool, seq
        if pool is not None:
            self.S, self.conv_tail = pool.S[seq], pool.conv[seq]
        else:
            self.S = torch.zeros(n_linear, n_heads, dk, dv, device=device, dtype=torch.float32)
            self.conv_tail = torch.zeros(n_linear, conv_k - 1, conv_dim, device=device, dtype=torch.float32)

    @property
    def length(self) -> int:
        return self.kv.length

    def advance(self, n: int) -> None:
        self.kv.advance(n)

    def reserve(self, end: int) -> None:
        self.kv.reserve(end)

    def free(self) -> None:
        if hasattr(self.kv, "free"):
            self.kv.free()
        if self.pool is not None:
            self.pool.release(self.seq)
            self.pool = None
            self.S = self.conv_tail = None
        elif self.seq is None:
            self.S.zero_()
            self.conv_tail.zero_()

    def bytes_used(self) -> int:
        return self.kv.bytes_used() + (self.S.numel() + self.conv_tail.numel()) * 4

    def fork(self) -> "HybridState":
        if self.pool is not None or not isinstance(self.kv, ContiguousKVCache):
            raise ValueError("fork() needs a standalone state with a contiguous KV cache")
        twin = HybridState.__new__(HybridState)
        twin.kv, twin.pool, twin.seq = self.kv.fork(), None, None
        twin.S, twin.conv_tail = self.S.clone(), self.conv_tail.clone()
        return twin


class HybridPool:
    """The paged KV pool plus one DeltaNet state slot per sequence (src/state.py:420-470):
    S [max_seqs, n_linear, H, dk, dv] fp32 and conv [max_seqs, n_linear, K-1, C] fp32, so one kernel launch per
    layer updates every sequence of a batch."""

    def __init__(self, kv: PagedKVPool, max_seqs: int, n_linear: int, n_heads: int, dk: int, dv: int,
                 conv_dim: int, conv_k: int, device="cpu"):
        self.kv = kv
        self.S = torch.zeros(max_seqs, n_linear, n_heads, dk, dv, device=device, dtype=torch.float32)
        self.conv = torch.zeros(max_seqs, n_linear, conv_k - 1, conv_dim, device=device, dtype=torch.float32)
        self.free_seqs = list(reversed(range(max_seqs)))
        self._seq_index: tuple[tuple, torch.Tensor | None] = ((), None)

    @property
    def allocator(self) -> BlockAllocator:
        return self.kv.allocator

    @property
    def block_size(self) -> int:
        return self.kv.block_size

    def blocks_for(self, n: int) -> int:
        return math.ceil(n / self.kv.block_size)

    @property
    def max_step_units(self) -> int:
        return 1

    @property
    def unit_bytes(self) -> int:
        return self.kv.unit_bytes

    def seq_index(self, states: list) -> torch.Tensor:
        """The states' slot numbers as a device int32 tensor, cached per batch composition."""
        key = tuple(st.seq for st in states)
        if self._seq_index[0] != key:
            self._seq_index = (key, to_device(torch.tensor(key, dtype=torch.int32), self.S.device))
        return self._seq_index[1]

    def new_sequence(self) -> HybridState:
        if not self.free_seqs:
            raise OutOfBlocks(f"all {self.S.shape[0]} sequence state slots are in use")
        return HybridState(self.kv.new_sequence(), pool=self, seq=self.free_seqs.pop())

    def release(self, seq: int) -> None:
        self.S[seq].zero_()
        self.conv[seq].zero_()
        self.free_seqs.append(seq)
