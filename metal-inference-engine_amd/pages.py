"""Device-resident paged-KV bookkeeping: block tables, lengths and the free-block stack in device memory
(librk_path.so rk_pages_*), the GPU counterpart of the engine's BlockAllocator / PagedSequence / batch_layout
(src/state.py:78-157, 182-186).

A decode step's layout -- the pool rows the new tokens are written to, each sequence's length after the step and its
block table -- comes from one small kernel (plus one for the tables when the batch rows are not the table's leading
rows), with no host work and no host-to-device copy: every step of a running batch can be replayed from one HIP
graph. The engine's own bookkeeping stays usable unchanged; this is for callers that want the step on the device.

Differences from the reference, by design: a failed step (too few free blocks, a row outside the table) takes
nothing for any sequence of the batch and sets a status word instead of raising at once; check() raises the
reference's exception (OutOfBlocks) from it. The blocks a successful step hands out, and their order, are the
reference's: block 0 first from a fresh pool, sequences in batch order, released blocks reused in table order.
"""
import torch

from native.rocm_native import load

STATUS = {1: "out of blocks", 2: "a sequence would outgrow its table row (max_blocks)",
          3: "a release would return more blocks than the pool has", 4: "a row index outside the table",
          5: "a row named twice in one step (a double allocation or a double free)"}


class OutOfBlocks(RuntimeError):
    """No free KV block is left for a step (the name of the reference's exception, src/state.py:74-75)."""


class DevicePages:
    """Block tables [max_seqs, max_blocks], lengths [max_seqs] and the free stack of a pool of num_blocks blocks, all
    int32 on `device`. Rows are sequence slots; the caller assigns them (e.g. a HybridPool's seq index)."""

    def __init__(self, num_blocks: int, max_seqs: int, max_blocks: int, block_size: int = 16, device="cuda"):
        self.num_blocks, self.max_seqs, self.max_blocks, self.block_size = num_blocks, max_seqs, max_blocks, block_size
        self.device = torch.device(device)
        i32 = dict(dtype=torch.int32, device=self.device)
        self.tables = torch.empty(max_seqs, max_blocks, **i32)
        self.lens = torch.empty(max_seqs, **i32)
        self.stack = torch.empty(num_blocks, **i32)
        self.meta = torch.empty(2, **i32)
        self.lib = load()
        self.lib.call("rk_pages_init", *self._state(), max_seqs, max_blocks, num_blocks, self._stream())

    def _state(self):
        return self.tables.data_ptr(), self.lens.data_ptr(), self.stack.data_ptr(), self.meta.data_ptr()

    def _stream(self) -> int:
        return torch.cuda.current_stream(self.device).cuda_stream

    def _rows(self, rows) -> torch.Tensor:
        if not isinstance(rows, torch.Tensor):
            rows = torch.tensor(list(rows), dtype=torch.int32)
        rows = rows.to(device=self.device, dtype=torch.int32).contiguous()
        if rows.dim() != 1 or not 1 <= rows.numel() <= 1024:
            raise ValueError(f"rows: 1 .. 1024 row indices, got shape {tuple(rows.shape)}")
        return rows

    def advance(self, rows, n_new: int = 1, slots=None, lens=None):
        """Grow sequences rows[b] (distinct) by n_new positions each, taking blocks as needed -> (slots int64
        [B * n_new]: block * block_size + offset of each new position, in batch order; lens int32 [B]: lengths after
        the step). Output tensors may be passed in (a captured graph reuses them)."""
        rows = self._rows(rows)
        B = rows.numel()
        if slots is None:
            slots = torch.empty(B * n_new, dtype=torch.int64, device=self.device)
        if lens is None:
            lens = torch.empty(B, dtype=torch.int32, device=self.device)
        if slots.numel() != B * n_new or lens.numel() != B:
            raise ValueError(f"advance: slots {slots.numel()} / lens {lens.numel()} for {B} rows x {n_new}")
        self.lib.call("rk_pages_advance", *self._state(), self.max_seqs, self.max_blocks, self.num_blocks,
                      self.block_size, rows.data_ptr(), B, int(n_new), slots.data_ptr(), lens.data_ptr(),
                      self._stream())
        return slots, lens

    def tables_for(self, rows, width: int | None = None, out=None) -> torch.Tensor:
        """The block tables of rows[b] as a [B, width] int32 tensor, 0 past the blocks each holds (width defaults to
        max_blocks): the `tables` argument of paged_attention."""
        rows = self._rows(rows)
        width = width or self.max_blocks
        if out is None:
            out = torch.empty(rows.numel(), width, dtype=torch.int32, device=self.device)
        self.lib.call("rk_pages_gather", self.tables.data_ptr(), self.lens.data_ptr(), self.max_seqs, self.max_blocks,
                      self.block_size, rows.data_ptr(), rows.numel(), width, out.data_ptr(), self._stream())
        return out

    def release(self, rows) -> None:
        """Return the blocks of rows[r] to the pool (reverse table order) and empty them."""
        rows = self._rows(rows)
        self.lib.call("rk_pages_release", *self._state(), self.max_seqs, self.max_blocks, self.num_blocks,
                      self.block_size, rows.data_ptr(), rows.numel(), self._stream())

    def status(self) -> int:
        """The status word (synchronises with the stream)."""
        return int(self.meta[1].item())

    def free_blocks(self) -> int:
        return int(self.meta[0].item())

    def check(self) -> None:
        """Raise for a failed step since the last check (OutOfBlocks for a lack of blocks), clearing the status."""
        st = self.status()
        if st:
            self.meta[1].zero_()
            if st == 1:
                raise OutOfBlocks(f"a step needed more than the {self.free_blocks()} free KV blocks")
            raise RuntimeError(f"paged KV bookkeeping: {STATUS.get(st, st)}")
