"""Paged KV scatter / gather on the GPU (rk_kv_write, rk_kv_gather) vs torch indexing on the CPU: bit-exact.

The state classes are the same on both sides; only the pool's device differs, so the CPU run is torch index_put /
advanced indexing (the reference's PagedKVPool.write_batch and PagedSequence.write / read, src/state.py:131-180) and
the GPU run is the HIP kernels.
"""
import pytest
import torch

from state import PagedKVPool

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def scrambled_pool(device, dtype, num_blocks=24, bs=4, Hkv=2, d=64):
    pool = PagedKVPool(2, Hkv, d, num_blocks, bs, device=device, dtype=dtype)
    taken = [pool.allocator.allocate() for _ in range(10)]
    pool.allocator.free([taken[i] for i in (7, 2, 9, 0, 5, 3, 8, 1, 6, 4)])   # recycled, non-monotonic tables
    return pool


@pytest.mark.parametrize("pool_dtype", [torch.float32, torch.bfloat16])
def test_sequence_write_then_read_matches_cpu(pool_dtype):
    gen = torch.Generator().manual_seed(0)
    cpu, gpu = scrambled_pool("cpu", pool_dtype), scrambled_pool(DEV, pool_dtype)
    seqs_c = [cpu.new_sequence() for _ in range(3)]
    seqs_g = [gpu.new_sequence() for _ in range(3)]
    for step, T in enumerate([5, 3, 9]):
        for sc, sg in zip(seqs_c, seqs_g):
            k = torch.randn(T, 2, 64, generator=gen) * 3
            v = torch.randn(T, 2, 64, generator=gen) * 3
            for layer in (0, 1):
                sc.write(layer, sc.length, k, v)
                sg.write(layer, sg.length, k.to(DEV), v.to(DEV))
            sc.advance(T)
            sg.advance(T)
    torch.cuda.synchronize()
    assert torch.equal(cpu.k.cpu(), gpu.k.cpu()) and torch.equal(cpu.v.cpu(), gpu.v.cpu())
    for sc, sg in zip(seqs_c, seqs_g):
        assert sc.block_table == sg.block_table
        for layer in (0, 1):
            for lo, end in ((0, sc.length), (3, sc.length), (5, 6), (4, 4)):
                kc, vc = sc.read(layer, end, lo)
                kg, vg = sg.read(layer, end, lo)
                assert kg.dtype == pool_dtype
                assert torch.equal(kc, kg.cpu()) and torch.equal(vc, vg.cpu())


@pytest.mark.parametrize("pool_dtype", [torch.float32, torch.bfloat16])
def test_batch_layout_write_batch_matches_cpu(pool_dtype):
    gen = torch.Generator().manual_seed(1)
    cpu, gpu = scrambled_pool("cpu", pool_dtype), scrambled_pool(DEV, pool_dtype)
    lens = [3, 4, 7]
    sc = [cpu.new_sequence() for _ in lens]
    sg = [gpu.new_sequence() for _ in lens]
    for a, b, n in zip(sc, sg, lens):
        a.reserve(n + 1); b.reserve(n + 1)
        a.length = b.length = n
    bc, oc, tc, lc = cpu.batch_layout(sc, lens)
    bg, og, tg, lg = gpu.batch_layout(sg, lens)
    assert torch.equal(tc, tg.cpu()) and torch.equal(lc, lg.cpu()) and tg.dtype == torch.int32
    k = torch.randn(3, 2, 64, generator=gen)
    v = torch.randn(3, 2, 64, generator=gen)
    cpu.write_batch(1, bc, oc, k, v)
    gpu.write_batch(1, bg, og, k.to(DEV), v.to(DEV))
    torch.cuda.synchronize()
    assert torch.equal(cpu.k.cpu(), gpu.k.cpu()) and torch.equal(cpu.v.cpu(), gpu.v.cpu())


def test_bf16_rounding_matches_torch():
    """fp32 -> bf16 in the scatter rounds to nearest even exactly as Tensor.to(torch.bfloat16), including ties,
    subnormals, infinities and NaN."""
    vals = torch.tensor([1.0, 1.00390625, 1.01171875, -2.5e-39, 3.4e38, float("inf"), -float("inf"), 0.0, -0.0,
                         1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, 65504.0, 1e-45] * 10)[:128]
    vals = torch.cat([vals, torch.randn(128)])          # 256 = one row of Hkv=1 x d=256
    pool = PagedKVPool(1, 1, 256, 2, 1, device=DEV, dtype=torch.bfloat16)
    slots = torch.tensor([1], dtype=torch.int64, device=DEV)
    pool.write_rows(0, slots, vals.view(1, 1, 256).to(DEV), vals.view(1, 1, 256).to(DEV))
    torch.cuda.synchronize()
    assert torch.equal(pool.k[0, 1, 0, 0].cpu().view(torch.int16), vals.to(torch.bfloat16).view(torch.int16))
