"""Paged KV scatter / gather on the GPU (rk_kv_write, rk_kv_gather) against the closed-form address map on the CPU,
bit-exact: position s of a sequence lives at pool[table[s // bs], s % bs] (src/kernels/attention.metal:115; the
writes of PagedKVPool.write_batch / PagedSequence.write and the gather of PagedSequence.read, src/state.py:131-180).
Tables are scattered, non-monotonic slices of a seeded permutation of the pool.
"""
import pytest
import torch

from native import kernels

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def address_map_write(pool, table, start, rows):
    """CPU reference: rows [n, Hkv, d] written at positions start .. start+n-1 (values rounded to the pool type)."""
    bs = pool.shape[1]
    for i in range(rows.shape[0]):
        s = start + i
        pool[int(table[s // bs]), s % bs] = rows[i].to(pool.dtype)


def address_map_read(pool, table, lo, end):
    bs = pool.shape[1]
    return torch.stack([pool[int(table[s // bs]), s % bs] for s in range(lo, end)]) if end > lo else pool[:0, 0]


@pytest.mark.parametrize("pool_dtype,bs", [(torch.float32, 4), (torch.bfloat16, 4), (torch.bfloat16, 16)])
def test_sequence_writes_then_reads_match_the_address_map(pool_dtype, bs):
    gen = torch.Generator().manual_seed(0)
    Hkv, d, NB = 2, 64, 40
    perm = torch.randperm(NB, generator=gen).to(torch.int32)
    tables = [perm[0:9], perm[9:20], perm[20:31]]               # 3 sequences, scattered blocks
    k_cpu = torch.full((NB, bs, Hkv, d), float("nan")).to(pool_dtype)
    v_cpu = k_cpu.clone()
    k_gpu, v_gpu = k_cpu.to(DEV), v_cpu.to(DEV)
    length = [0, 0, 0]
    for T in (5, 3, 9):                                           # chunks of T tokens per sequence
        for i, tab in enumerate(tables):
            k = torch.randn(T, Hkv, d, generator=gen) * 3
            v = torch.randn(T, Hkv, d, generator=gen) * 3
            address_map_write(k_cpu, tab, length[i], k)
            address_map_write(v_cpu, tab, length[i], v)
            pos = torch.arange(length[i], length[i] + T)
            slots = tab[pos // bs].long() * bs + pos % bs
            kernels.kv_write(k_gpu, v_gpu, slots.to(DEV), k.to(DEV), v.to(DEV))
            length[i] += T
    torch.cuda.synchronize()
    assert torch.equal(k_cpu.float().nan_to_num(7.0),
                       k_gpu.cpu().float().nan_to_num(7.0))
    assert torch.equal(v_cpu.float().nan_to_num(7.0), v_gpu.cpu().float().nan_to_num(7.0))
    for i, tab in enumerate(tables):
        for lo, end in ((0, length[i]), (3, length[i]), (5, 6), (4, 4)):
            kg, vg = kernels.kv_gather(k_gpu, v_gpu, tab.to(DEV), lo, end)
            assert kg.dtype == pool_dtype
            assert torch.equal(kg.cpu(), address_map_read(k_cpu, tab, lo, end))
            assert torch.equal(vg.cpu(), address_map_read(v_cpu, tab, lo, end))


@pytest.mark.parametrize("pool_dtype", [torch.float32, torch.bfloat16])
def test_decode_step_write_matches_the_address_map(pool_dtype):
    """One new token per sequence at position lens[i] (a decode step's write_batch), into a 2-layer pool: only the
    addressed rows of the addressed layer change."""
    gen = torch.Generator().manual_seed(1)
    bs, Hkv, d, NB = 4, 2, 64, 24
    lens = [3, 4, 7]
    perm = torch.randperm(NB, generator=gen).to(torch.int32)
    tables = torch.zeros(3, 2, dtype=torch.int32)
    tables[0, :1], tables[1, :2], tables[2, :2] = perm[:1], perm[1:3], perm[3:5]
    both = torch.randn(2, 2, NB, bs, Hkv, d, generator=gen).to(pool_dtype)
    k_cpu, v_cpu = both[0].clone(), both[1].clone()
    k_gpu, v_gpu = k_cpu.to(DEV), v_cpu.to(DEV)
    k = torch.randn(3, Hkv, d, generator=gen)
    v = torch.randn(3, Hkv, d, generator=gen)
    for i, p in enumerate(lens):
        k_cpu[1, int(tables[i, p // bs]), p % bs] = k[i].to(pool_dtype)
        v_cpu[1, int(tables[i, p // bs]), p % bs] = v[i].to(pool_dtype)
    slots = torch.tensor([int(tables[i, p // bs]) * bs + p % bs for i, p in enumerate(lens)])
    kernels.kv_write(k_gpu[1], v_gpu[1], slots.to(DEV), k.to(DEV), v.to(DEV))
    torch.cuda.synchronize()
    assert torch.equal(k_cpu, k_gpu.cpu()) and torch.equal(v_cpu, v_gpu.cpu())


def test_bf16_rounding_matches_torch():
    """fp32 -> bf16 in the scatter rounds to nearest even exactly as Tensor.to(torch.bfloat16), including ties,
    subnormals, infinities and NaN."""
    vals = torch.tensor([1.0, 1.00390625, 1.01171875, -2.5e-39, 3.4e38, float("inf"), -float("inf"), 0.0, -0.0,
                         1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, 65504.0, 1e-45] * 10)[:128]
    vals = torch.cat([vals, torch.randn(128)])          # 256 = one row of Hkv=1 x d=256
    k = torch.zeros(2, 1, 1, 256, dtype=torch.bfloat16, device=DEV)
    v = torch.zeros_like(k)
    slots = torch.tensor([1], dtype=torch.int64, device=DEV)
    kernels.kv_write(k, v, slots, vals.view(1, 1, 256).to(DEV), vals.view(1, 1, 256).to(DEV))
    torch.cuda.synchronize()
    assert torch.equal(k[1, 0, 0].cpu().view(torch.int16), vals.to(torch.bfloat16).view(torch.int16))
