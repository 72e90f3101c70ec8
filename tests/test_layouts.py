"""The layout builders the workloads and GPU tests use (workloads.py), on the CPU: scattered tables cover each
sequence with distinct blocks of the pool; ring tables name, for every block of a window, the ring unit a
block-by-block write of the whole history left that block in (simulated here with a dict of unit -> block), and
unit 0 below the window; the prefill attention's work list covers every query block once, whole or as pieces cut at
absolute tile multiples."""
import math

import pytest
import torch

import workloads as wl


def test_scattered_tables_are_distinct_and_padded():
    gen = torch.Generator().manual_seed(0)
    lens = [1, 16, 17, 300, 0 + 5]
    t = wl.scattered_tables(lens, 40, 16, gen)
    used = []
    for row, n in zip(t.tolist(), lens):
        nb = math.ceil(n / 16)
        used += row[:nb]
        assert all(x == 0 for x in row[nb:])
    assert len(set(used)) == len(used) and all(0 <= x < 40 for x in used)
    with pytest.raises(ValueError):
        wl.scattered_tables([16 * 41], 40, 16, gen)


@pytest.mark.parametrize("W,bs,chunk", [(37, 4, 16), (100, 16, 16), (4096, 16, 512), (5, 1, 3)])
def test_ring_tables_name_the_unit_holding_each_window_block(W, bs, chunk):
    gen = torch.Generator().manual_seed(W)
    lens = [1, 2, W - 1, W, W + 1, 2 * W + 5, 3 * W + 33, 7 * W + 1]
    ring = wl.ring_size(W, bs, chunk)
    tables, units, rings = wl.ring_tables(lens, W, bs, ring, gen)
    owned = [u for r in rings for u in r]
    assert 0 not in owned and len(set(owned)) == len(owned) and max(owned) < units
    for i, n in enumerate(lens):
        holds = {}                                        # unit -> logical block it holds after the writes
        for b in range(math.ceil(n / bs)):
            holds[rings[i][b % ring]] = b
        first = max(0, n - W) // bs
        row = tables[i].tolist()
        for b in range(math.ceil(n / bs)):
            if b < first:
                assert row[b] == 0
            else:
                assert holds[row[b]] == b                 # the window's block is still in the ring
        # a chunk of up to `chunk` tokens after the window still fits (the ring-size rule)
        span = math.ceil((n + chunk) / bs) - max(0, n - W + 1) // bs
        assert span <= ring


# ---------------------------------------------------------------- the CPU model of the device page table

def test_pages_model_known_answers():
    """The reference allocator's documented behaviour (src/state.py:78-103): a fresh pool hands out block 0 first,
    in ascending order; freed blocks come back in the order the table held them; growth takes only missing blocks."""
    from oracle.pages_ref import PagesModel
    m = PagesModel(num_blocks=10, max_seqs=4, max_blocks=5, block_size=4)
    assert m.advance([0], 9) == ([0, 1, 2, 3, 4, 5, 6, 7, 8], [9])          # blocks 0, 1, 2
    assert m.tables[0] == [0, 1, 2]
    assert m.advance([1, 0], 1) == ([12, 9], [1, 10])                       # seq 1 takes block 3; seq 0 fits in 2
    assert m.tables[1] == [3]
    m.release([0])
    assert m.advance([2], 6) == ([0, 1, 2, 3, 4, 5], [6])                    # blocks 0, 1 again, in table order
    assert m.tables[2] == [0, 1] and len(m.free) == 10 - 3                  # blocks 3 (seq 1), 0, 1 (seq 2)


def test_pages_model_all_or_nothing():
    from oracle.pages_ref import PagesModel
    m = PagesModel(num_blocks=3, max_seqs=3, max_blocks=8, block_size=2)
    assert m.advance([0], 4) is not None                                     # 2 blocks taken, 1 free
    before = ([list(t) for t in m.tables], list(m.lens), list(m.free))
    assert m.advance([1, 2], 1) is None and m.status == 1                    # needs 2, 1 free: nothing moves
    assert ([list(t) for t in m.tables], list(m.lens), list(m.free)) == before
    m.status = 0
    assert m.advance([0], 100) is None and m.status == 2                     # past max_blocks
    assert m.advance([5], 1) is None and m.status == 4                       # no such row


@pytest.mark.parametrize("split", [0, 1, 2, 5, 320])
@pytest.mark.parametrize("window,causal", [(None, True), (40, True), (None, False)])
def test_prefill_work_covers_every_block_once(split, window, causal):
    """rk_paged_prefill's work list: every (segment, block) appears as one whole entry or as pieces over consecutive
    disjoint tile ranges that together are exactly the block's range, cut at absolute multiples of `split`; the
    pieces of a block use consecutive slots; entries go longest first."""
    from native import kernels
    lengths, starts = [70, 129, 3, 40, 1], [50, 900, 500, 0, 7]
    work, n_slots = kernels.prefill_work(lengths, starts, window, causal, split)
    entries = [work[i:i + 5] for i in range(0, len(work), 5)]
    sizes = [e[2] - e[1] for e in entries]
    assert sizes == sorted(sizes, reverse=True) and min(sizes) >= 1
    by_block, slots = {}, []
    for word, t0, t1, first, pp in entries:
        by_block.setdefault(word, []).append((t0, t1, first, pp >> 16, pp & 0xffff))
    for s, (n, p) in enumerate(zip(lengths, starts)):
        for qb in range(-(-n // 32)):
            hi = p + min(n, 32 * (qb + 1)) if causal else p + n
            lo = max(0, p + 32 * qb - window + 1) if window else 0
            got = sorted(by_block.pop((s << 16) | qb))
            assert got[0][0] == lo // 32 and got[-1][1] == -(-hi // 32)
            if len(got) == 1:
                assert got[0][2] == -1 and got[0][4] == 1
                continue
            assert all(a[1] == b[0] for a, b in zip(got, got[1:]))          # consecutive, disjoint
            assert all(c[0] % split == 0 for c in got[1:])                  # cut at absolute multiples
            first = got[0][2]
            assert [(c[2], c[3], c[4]) for c in got] == [(first, i, len(got)) for i in range(len(got))]
            slots.extend(range(first, first + len(got)))
    assert not by_block
    assert sorted(slots) == list(range(n_slots))


def test_prefill_auto_split():
    """The automatic split size: none while the 32-query blocks times the KV heads give every CU a workgroup (a
    packed batch like config 5); for one chunk over a long prefix, pieces that bring the workgroups to about one
    per CU, never smaller than the minimum piece."""
    from native import kernels
    assert kernels.prefill_split_tiles([500] * 128, 2, 256) == 0           # 256 workgroups already
    assert kernels.prefill_split_tiles([], 2, 256) == 0
    assert kernels.prefill_split_tiles([10] * 4, 2, 256) == kernels.PREFILL_MIN_SPLIT
    spans = [1024 + i for i in range(16)]                                   # 512 queries after a 32K prefix
    size = kernels.prefill_split_tiles(spans, 2, 256)
    assert size == -(-sum(spans) * 2 // 256)
    work, n_slots = kernels.prefill_work([512], [32768], None, True, None, 2, 256)
    n = len(work) // 5
    assert 256 <= 2 * n <= 2 * 256 + 2 * 16 and n_slots == n               # every block split, ~1 piece per CU
    gen = torch.Generator().manual_seed(5)                                  # config 5's draw
    lengths = torch.randint(64, 2049, (8,), generator=gen).tolist()
    starts = torch.randint(0, 16385, (8,), generator=gen).tolist()
    assert kernels.prefill_work(lengths, starts, None, True, None, 2, 256)[1] == 0   # config 5: not split


def test_prefill_balance_split():
    """The balance split of the fp32-operand kernel: with enough workgroups to fill the CUs, blocks longer than a
    quarter of a CU's share of the tiles are cut to that size (never below two minimum pieces), and nothing is cut
    when every block is already that short."""
    from native import kernels
    gen = torch.Generator().manual_seed(5)                                  # config 5's draw
    lengths = torch.randint(64, 2049, (8,), generator=gen).tolist()
    starts = torch.randint(0, 16385, (8,), generator=gen).tolist()
    spans = [-(-(p + min(n, (qb + 1) * 32)) // 32) for n, p in zip(lengths, starts) for qb in range(-(-n // 32))]
    size = kernels.prefill_split_tiles(spans, 2, 256, balance=True)
    assert size == max(2 * kernels.PREFILL_MIN_SPLIT, -(-sum(spans) * 2 // (256 * kernels.PREFILL_BALANCE_PIECES)))
    assert 0 < size < max(spans)
    assert kernels.prefill_split_tiles(spans, 2, 256) == 0                  # the bf16-operand kernel: not split
    work, n_slots = kernels.prefill_work(lengths, starts, None, True, None, 2, 256, balance=True)
    ents = [work[i:i + 5] for i in range(0, len(work), 5)]
    assert n_slots > 0 and max(e[2] - e[1] for e in ents) <= size
    assert sum(e[2] - e[1] for e in ents) == sum(spans)                      # every tile once
    assert kernels.prefill_split_tiles([100] * 1000, 2, 256, balance=True) == 0      # short blocks stay whole
    # too few workgroups: the one-piece-per-CU rule holds with or without balance
    assert kernels.prefill_split_tiles([1024] * 16, 2, 256, balance=True) == kernels.prefill_split_tiles([1024] * 16, 2, 256)


def test_prefill_block_index_division():
    """The prefill kernels' block index pos // bs without a divide: the fp32-operand kernel takes mulhi(pos,
    floor((2^32 - 1) / bs)) plus one correction, exact for every pos < 2^32 and bs >= 1; the bf16-operand kernel
    takes mulhi(pos, ceil(2^32 / bs)) alone, exact while pos * bs < 2^32, and only for bs >= 2 (the reciprocal of 1
    does not fit 32 bits). Checked over block sizes 1 .. 4096 at edge and random positions."""
    import numpy as np
    rng = np.random.default_rng(5)
    for bs in list(range(1, 130)) + [255, 256, 1000, 1024, 4095, 4096, 65535, 65536, 70003]:
        lo = (2 ** 32 - 1) // bs
        edge = [0, 1, bs - 1, bs, bs + 1, 2 ** 31 - 1, 2 ** 31 - bs, (2 ** 31 - 1) // bs * bs]
        pos = np.array(edge + rng.integers(0, 2 ** 31, 2000).tolist(), dtype=np.uint64)
        q = (pos * np.uint64(lo)) >> np.uint64(32)
        r = pos - q * np.uint64(bs)
        q = q + (r >= bs)
        assert np.array_equal(q, pos // np.uint64(bs)), bs
        if bs >= 2:
            up = (2 ** 32 - 1) // bs + 1
            assert up < 2 ** 32
            ok = pos[pos * np.uint64(bs) < np.uint64(2 ** 32)]
            assert np.array_equal((ok * np.uint64(up)) >> np.uint64(32), ok // np.uint64(bs)), bs
    assert (2 ** 32 - 1) // 1 + 1 == 2 ** 32                    # bs = 1: the rounded-up reciprocal overflows
