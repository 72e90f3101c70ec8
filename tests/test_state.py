"""State layout and host logic on the CPU (the reference's tests/test_paged.py:24-108 checks that do not need model
weights): allocator order and refusals, all-or-nothing growth, non-monotonic recycled tables, paged == contiguous
storage, batch_layout padding and dtypes, DeltaNet slot reuse zeroed, byte accounting."""
import pytest
import torch

from state import BlockAllocator, ContiguousKVCache, HybridPool, HybridState, OutOfBlocks, PagedKVPool, kv_buffers


def test_allocator_order_and_refusals():
    a = BlockAllocator(4)
    got = [a.allocate() for _ in range(4)]
    assert got == [0, 1, 2, 3] and a.num_free == 0
    with pytest.raises(OutOfBlocks):
        a.allocate()
    a.free(got[:2])
    assert a.num_free == 2 and {a.allocate(), a.allocate()} == {0, 1}
    with pytest.raises(ValueError):
        a.free([7])                      # never handed out
    a.free([3])
    with pytest.raises(ValueError):
        a.free([3])                      # twice
    with pytest.raises(ValueError):
        a.free([2, 2])


def test_kv_buffers_are_halves_of_one_allocation():
    k, v = kv_buffers((3, 4, 2, 8), "cpu", torch.bfloat16)
    assert k.is_contiguous() and v.is_contiguous() and k.untyped_storage().data_ptr() == v.untyped_storage().data_ptr()
    assert v.data_ptr() - k.data_ptr() == k.numel() * 2 and float(k.abs().sum()) == 0


def recycled_pool(num_blocks=64, bs=4, dtype=torch.float32):
    pool = PagedKVPool(2, 2, 8, num_blocks, bs, dtype=dtype)
    taken = [pool.allocator.allocate() for _ in range(10)]
    pool.allocator.free([taken[i] for i in (7, 2, 9, 0, 5, 3, 8, 1, 6, 4)])
    return pool


def test_paged_storage_equals_contiguous():
    gen = torch.Generator().manual_seed(0)
    pool = recycled_pool()
    seq = pool.new_sequence()
    ref = ContiguousKVCache(2, 2, 8, 64)
    for T in (5, 1, 1, 9, 3):
        k, v = torch.randn(T, 2, 8, generator=gen), torch.randn(T, 2, 8, generator=gen)
        for layer in (0, 1):
            seq.write(layer, seq.length, k, v)
            ref.write(layer, ref.length, k, v)
        seq.advance(T)
        ref.advance(T)
    assert len(seq.block_table) == -(-seq.length // 4) and seq.block_table != sorted(seq.block_table)
    for layer in (0, 1):
        for lo in (0, 3, 8):
            kp, vp = seq.read(layer, seq.length, lo)
            kc, vc = ref.read(layer, ref.length, lo)
            assert torch.equal(kp, kc) and torch.equal(vp, vc)


def test_growth_is_all_or_nothing():
    pool = PagedKVPool(1, 2, 8, 4, 4)
    a, b = pool.new_sequence(), pool.new_sequence()
    a.reserve(4)
    with pytest.raises(OutOfBlocks):
        b.reserve(20)                      # 5 blocks, 3 free
    assert b.block_table == [] and pool.allocator.num_free == 3
    b.reserve(12)
    assert len(b.block_table) == 3 and pool.allocator.num_free == 0
    a.free()
    b.free()
    assert pool.allocator.num_free == 4


def test_batch_layout():
    pool = recycled_pool()
    seqs = [pool.new_sequence() for _ in range(3)]
    starts = [0, 5, 12]
    for s, p in zip(seqs, starts):
        s.reserve(p + 1)
    blocks, offsets, tables, lens = pool.batch_layout(seqs, starts)
    assert tables.dtype == torch.int32 and lens.dtype == torch.int32 and blocks.dtype == torch.int64
    assert lens.tolist() == [1, 6, 13] and offsets.tolist() == [0, 1, 0]
    width = max(len(s.block_table) for s in seqs)
    for i, s in enumerate(seqs):
        assert tables[i].tolist() == s.block_table + [0] * (width - len(s.block_table))
        assert int(blocks[i]) == s.block_table[starts[i] // 4]
    k = torch.randn(3, 2, 8)
    pool.write_batch(1, blocks, offsets, k, -k)
    for i, s in enumerate(seqs):
        kk, vv = s.read(1, starts[i] + 1)
        assert torch.equal(kk[-1], k[i]) and torch.equal(vv[-1], -k[i])


def test_hybrid_pool_slots():
    kv = PagedKVPool(1, 2, 8, 16, 4)
    pool = HybridPool(kv, 2, 3, 2, 4, 4, 24, 4)
    assert pool.S.shape == (2, 3, 2, 4, 4) and pool.conv.shape == (2, 3, 3, 24)
    a, b = pool.new_sequence(), pool.new_sequence()
    assert (a.seq, b.seq) == (0, 1)
    with pytest.raises(OutOfBlocks):
        pool.new_sequence()
    a.S.fill_(1.0)
    a.conv_tail.fill_(2.0)
    idx = pool.seq_index([b, a])
    assert idx.tolist() == [1, 0] and idx.dtype == torch.int32 and pool.seq_index([b, a]) is idx
    a.kv.reserve(9)
    a.free()
    assert a.S is None and pool.allocator.num_free == 16
    c = pool.new_sequence()
    assert c.seq == 0 and float(c.S.abs().sum()) == 0 and float(c.conv_tail.abs().sum()) == 0


def test_bytes_accounting():
    kv = PagedKVPool(2, 2, 8, 16, 4)
    pool = HybridPool(kv, 2, 3, 2, 4, 4, 24, 4)
    st = pool.new_sequence()
    st.kv.reserve(9)
    per_block = 2 * 2 * 4 * 2 * 8 * 4          # K and V, 2 layers, 4 positions, 2 heads x 8, fp32
    fixed = (3 * 2 * 4 * 4 + 3 * 3 * 24) * 4
    assert st.bytes_used() == 3 * per_block + fixed


def test_standalone_state_fork_and_free():
    st = HybridState(ContiguousKVCache(1, 2, 8, 32), 2, 2, 4, 4, 24, 4)
    st.S.fill_(3.0)
    st.kv.write(0, 0, torch.ones(5, 2, 8), torch.ones(5, 2, 8))
    st.kv.advance(5)
    twin = st.fork()
    twin.S.zero_()
    assert float(st.S.sum()) > 0 and twin.length == 5
    st.free()
    assert float(st.S.abs().sum()) == 0


# ---------------------------------------------------------------- grouped pool with sliding-window rings

def test_grouped_pool_random_chunks_against_a_dict_oracle():
    """Random chunk schedules up to max_chunk over 8 layers (6 sliding, 2 full): every read of a layer's window
    returns exactly what was written at those positions, stale ring slots are NaN-poisoned yet never read, every
    group holds exactly min(R, blocks) / blocks units, an oversized chunk is refused, and free returns every unit."""
    import random
    from state import GroupedKVPool
    rnd = random.Random(1)
    for W, bs, C in ((8, 4, 3), (8, 4, 7), (6, 3, 4), (5, 4, 4), (5, 3, 7), (16, 16, 16)):
        layers = [W, W, W, None] * 2
        pool = GroupedKVPool(layers, 1, 2, num_blocks=64, block_size=bs, max_chunk=C, poison=True)
        assert pool.groups == [[3, 7], [0, 1], [2, 4], [5, 6]] and pool.sliding == [False, True, True, True]
        seq, written, pos = pool.new_sequence(), {}, 0
        for _ in range(30):
            n = rnd.randint(1, C)
            seq.check_forward(pos, pos + n)
            for layer, w in enumerate(layers):
                k, v = torch.randn(n, 1, 2), torch.randn(n, 1, 2)
                seq.write(layer, pos, k, v)
                for j in range(n):
                    written[layer, pos + j] = (k[j], v[j])
                lo = max(0, pos - w + 1) if w else 0
                K, V = seq.read(layer, pos + n, lo)
                assert torch.equal(K, torch.stack([written[layer, t][0] for t in range(lo, pos + n)]))
                assert torch.equal(V, torch.stack([written[layer, t][1] for t in range(lo, pos + n)]))
            seq.advance(n)
            pos += n
            nb = -(-pos // bs)
            assert [len(t) for t in seq.tables] == [min(pool.ring, nb) if sl else nb for sl in pool.sliding]
            assert pool.allocator.num_free + sum(map(len, seq.tables)) == pool.allocator.num_blocks
        with pytest.raises(ValueError):
            seq.check_forward(pos, pos + C + bs + W)
        seq.free()
        assert pool.allocator.num_free == pool.allocator.num_blocks


def test_grouped_pool_reserve_is_all_or_nothing():
    from state import GroupedKVPool, OutOfBlocks
    pool = GroupedKVPool([8, 8, 8, None] * 2, 1, 2, num_blocks=3, block_size=4, max_chunk=4)
    a, b = pool.new_sequence(), pool.new_sequence()
    a.reserve(8)
    with pytest.raises(OutOfBlocks):
        b.reserve(12)
    assert b.tables == [[], [], [], []] and pool.allocator.num_free == 4
    assert pool.blocks_for(8) == 8 and pool.blocks_for(100) == 25 + 3 * pool.ring


def test_grouped_batch_layout_and_windowed_decode_on_the_cpu():
    """batch_layout of a sliding group: entries before the window are pad_block, the new token's unit is retagged
    (poisoned when it takes a new block), and the oracle's windowed paged attention over those tables, with every
    stale slot NaN, equals attention over exactly the window's positions."""
    from oracle import backend_ref, ops_ref
    from state import GroupedKVPool
    W, bs, Hq, Hkv, d = 10, 4, 4, 2, 8
    pool = GroupedKVPool([W, None], Hkv, d, num_blocks=64, block_size=bs, max_chunk=4, poison=True)
    g_sl, slot = pool.layer_map[0]
    assert pool.sliding[g_sl]
    lens = [1, 5, 11, 23, 40]
    seqs, hist = [pool.new_sequence() for _ in lens], []
    gen = torch.Generator().manual_seed(3)
    for s, n in zip(seqs, lens):                    # history of n - 1 tokens written in chunks of <= max_chunk
        K, V = torch.randn(n, Hkv, d, generator=gen), torch.randn(n, Hkv, d, generator=gen)
        for t in range(0, n - 1, 4):
            e = min(n - 1, t + 4)
            s.check_forward(t, e)
            s.write(0, t, K[t:e], V[t:e])
            s.advance(e - t)
        hist.append((K, V))
    starts = [n - 1 for n in lens]
    for s, p in zip(seqs, starts):
        s.reserve(p + 1)
    blocks, offsets, tables, lens_t = pool.batch_layout(seqs, starts)
    for i, (s, p) in enumerate(zip(seqs, starts)):
        first = max(0, p + 1 - W) // bs
        assert tables[g_sl, i, :first].tolist() == [pool.pad_block] * first
        assert int(blocks[g_sl, i]) == s.unit(g_sl, p // bs)
    k_new = torch.stack([K[-1] for K, _ in hist])
    v_new = torch.stack([V[-1] for _, V in hist])
    pool.write_batch(slot, blocks[g_sl], offsets, k_new, v_new)
    q = torch.randn(len(lens), Hq, d, generator=gen)
    out = backend_ref.paged_attention(q, pool.k[slot], pool.v[slot], tables[g_sl], lens_t, bs, window=W)
    assert torch.isfinite(out).all()
    want = torch.cat([ops_ref.attention(q[i:i + 1], K[max(0, n - W):], V[max(0, n - W):])
                      for i, ((K, V), n) in enumerate(zip(hist, lens))])
    assert torch.allclose(out, want, rtol=0, atol=1e-6)
