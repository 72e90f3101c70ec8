"""P1 parity: HIP paged decode attention (rk_paged_decode) vs the CPU oracle (TorchBackend.paged_attention restated).

Cases follow the reference's kernel tests (tests/test_kernels.py:106-198): scrambled block tables over lengths
[1, 7, 16, 33, 300] at 8/2 x 256, 14/2 x 64 and 16/4 x 128 heads; a bf16 pool equal, bit for bit, to the fp32 kernel
on the widened pool; q-scale 30 (scores past exp's range without a max subtraction); sliding windows with the blocks
before each window NaN-poisoned; refusal of other KV dtypes. Plus BASELINE configs 1 and 3 at full size.
Tolerances: fp32 within 1e-5 relative (max|diff| / max|ref|); bf16 pools are compared with the oracle run on the
widened pool, where the kernel's arithmetic is fp32, so the same 1e-5 applies (the north-star bar for bf16 outputs is
1e-2).
"""
import pytest
import torch

import workloads as wl
from helpers import rel_err
from oracle import backend_ref

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
REF_LENS = [1, 7, 16, 33, 300]


def gpu(backend, case, gate=False):
    c = case.to(DEV)
    out = backend.paged_attention(c.q, c.k_pool, c.v_pool, c.tables, c.lens, c.block_size, c.window,
                                  gate=c.gate if gate else None)
    torch.cuda.synchronize()
    return out.cpu()


def oracle(case, gate=False):
    f = lambda t: t.float() if t.is_floating_point() else t
    o = backend_ref.paged_attention(case.q, f(case.k_pool), f(case.v_pool), case.tables, case.lens, case.block_size,
                                    case.window)
    return backend_ref.gate(o, case.gate) if gate else o


def test_config1_fp32_with_gate(backend):
    case = wl.c1_paged_decode()
    got, want = gpu(backend, case, gate=True), oracle(case, gate=True)
    print(f"config 1: rel err {rel_err(got, want):.2e}")
    assert rel_err(got, want) < 1e-5


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("Hq,Hkv,d", [(8, 2, 256), (14, 2, 64), (16, 4, 128)])
def test_reference_lengths(backend, Hq, Hkv, d, dtype):
    case = wl.paged_decode_case(REF_LENS, 32, Hq, Hkv, d, 16, dtype, seed=11)
    got, want = gpu(backend, case), oracle(case)
    assert torch.isfinite(got).all()
    assert rel_err(got, want) < 1e-5


@pytest.mark.parametrize("Hq,Hkv,d", [(8, 2, 256), (16, 4, 128), (14, 2, 64)])
def test_bf16_pool_equals_fp32_kernel_on_widened_pool(backend, Hq, Hkv, d):
    case = wl.paged_decode_case(REF_LENS, 32, Hq, Hkv, d, 16, torch.bfloat16, seed=12)
    wide = wl.PagedDecodeCase(case.q, case.gate, case.k_pool.float(), case.v_pool.float(), case.tables, case.lens,
                              case.block_size)
    assert torch.equal(gpu(backend, case), gpu(backend, wide))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_large_scores_stay_finite(backend, dtype):
    case = wl.paged_decode_case([300, 2048, 5], 160, 8, 2, 256, 16, dtype, seed=13, q_scale=30.0)
    got, want = gpu(backend, case), oracle(case)
    assert torch.isfinite(got).all()
    assert rel_err(got, want) < 1e-5


@pytest.mark.parametrize("block_size", [1, 4, 16, 32])
def test_other_block_sizes(backend, block_size):
    lens = [5, 37, 64, 100]
    nb = sum(-(-n // block_size) for n in lens) + 3
    case = wl.paged_decode_case(lens, nb, 8, 2, 128, block_size, torch.float32, seed=14)
    assert rel_err(gpu(backend, case), oracle(case)) < 1e-5


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("W", [16, 20, 128])
def test_window_never_reads_blocks_before_it(backend, dtype, W):
    lens = [1, W, W + 1, 2 * W + 3, 300]
    nbs = [-(-n // 16) for n in lens]
    case = wl.paged_decode_case(lens, sum(nbs), 16, 4, 128, 16, dtype, seed=15, window=W)
    want = oracle(case)                                   # before any poisoning
    for i, n in enumerate(lens):
        for j in range(max(0, n - W) // 16):              # blocks wholly before the window
            blk = int(case.tables[i, j])
            case.k_pool[blk] = float("nan")
            case.v_pool[blk] = float("nan")
    got = gpu(backend, case)
    assert torch.isfinite(got).all()
    assert rel_err(got, want) < 1e-5


def test_config3_full_size(backend):
    case = wl.c3_paged_decode()
    got, want = gpu(backend, case, gate=True), oracle(case, gate=True)
    err = rel_err(got, want)
    print(f"config 3: {case.q.shape[0]} sequences, {int(case.lens.sum())} positions, rel err {err:.2e}")
    assert err < 1e-5


@pytest.mark.parametrize("S", [1, 5, 300, 2048])
def test_contiguous_decode_attention(backend, S):
    gen = torch.Generator().manual_seed(S)
    q = torch.randn(1, 8, 256, generator=gen)
    k, v = torch.randn(S, 2, 256, generator=gen), torch.randn(S, 2, 256, generator=gen)
    from oracle import ops_ref
    want = ops_ref.attention(q, k, v, causal=True)
    got = backend.attention(q.to(DEV), k.to(DEV), v.to(DEV)).cpu()
    if S == 1:                                            # one key: the output is that key's value, exactly
        assert torch.equal(got, v.repeat_interleave(4, dim=1))
    assert rel_err(got, want) < 1e-5


@pytest.mark.parametrize("S,W", [(15, 16), (16, 16), (17, 16), (35, 16), (4097, 4096), (8192, 4096)])
def test_contiguous_window(backend, S, W):
    gen = torch.Generator().manual_seed(S + W)
    q = torch.randn(1, 16, 128, generator=gen)
    k, v = (torch.randn(S, 4, 128, generator=gen).to(torch.bfloat16) for _ in range(2))
    from oracle import ops_ref
    want = ops_ref.attention(q, k.float(), v.float(), window=W)
    got = backend.attention(q.to(DEV), k.to(DEV), v.to(DEV), window=W).cpu()
    assert rel_err(got, want) < 1e-5


@pytest.mark.parametrize("kd,vd", [(torch.float16, torch.float16), (torch.bfloat16, torch.float32)])
def test_other_kv_dtypes_refused(backend, kd, vd):
    case = wl.paged_decode_case(REF_LENS, 32, 8, 2, 256, 16, torch.float32, seed=16).to(DEV)
    with pytest.raises(TypeError):
        backend.paged_attention(case.q, case.k_pool.to(kd), case.v_pool.to(vd), case.tables, case.lens, 16)


def test_stale_workspace_is_never_read(backend):
    """With more split workgroups than tiles (REF_LENS: 25 tiles), empty ranges write no partial; the merge must not
    read their slots. The workspace is filled with NaN first: the output must still match the oracle."""
    from native import kernels
    case = wl.paged_decode_case(REF_LENS, 32, 8, 2, 256, 16, torch.bfloat16, seed=13)
    c = case.to(DEV)
    lib = backend.lib
    need = lib.lib.rk_paged_decode_workspace_bytes(len(REF_LENS), 8, 2, 256, 16, c.tables.shape[1])
    kernels.workspace(c.q.device, need).view(torch.float32).fill_(float("nan"))
    got = gpu(backend, case, gate=True)
    assert torch.isfinite(got).all()
    assert rel_err(got, oracle(case, gate=True)) < 1e-5


def test_ranges_cut_by_cost_with_empty_and_short_sequences(backend):
    """With at least 16 tiles per split workgroup the ranges are cut by cost (tiles plus a fixed cost per sequence):
    here 20 sequences with empty, 1-33-position and long ones between each other, ~4,700 tiles over 256 workgroups.
    The merge must find each sequence's workgroups under that cut, skip the ones whose range holds only another
    sequence's cost units, and never read a slot no workgroup wrote (the workspace is NaN-filled first)."""
    from native import kernels
    lens = [0, 9000, 1, 0, 7000, 17, 0, 12000, 300, 0, 9000, 16, 8192, 0, 2, 11000, 33, 0, 9500, 5]
    assert sum((n + 15) // 16 for n in lens) >= 16 * 256
    case = wl.paged_decode_case(lens, 6000, 8, 2, 256, 16, torch.bfloat16, seed=19)
    c = case.to(DEV)
    need = backend.lib.lib.rk_paged_decode_workspace_bytes(len(lens), 8, 2, 256, 16, c.tables.shape[1])
    kernels.workspace(c.q.device, need).view(torch.float32).fill_(float("nan"))
    got = gpu(backend, case, gate=True)
    assert torch.isfinite(got).all()
    live = [i for i, n in enumerate(lens) if n > 0]        # the oracle, like ops.attention, needs a key
    assert torch.equal(got[[i for i, n in enumerate(lens) if n == 0]], torch.zeros(lens.count(0), 8, 256))
    sub = wl.PagedDecodeCase(case.q[live], case.gate[live], case.k_pool, case.v_pool, case.tables[live],
                             case.lens[live], case.block_size)
    assert rel_err(got[live], oracle(sub, gate=True)) < 1e-5


def planned(backend, case, gate=True):
    """The same call with the batch layout plan made first (rk_paged_decode_plan -> rk_paged_decode_planned)."""
    c = case.to(DEV)
    NB, bs, Hkv, d = c.k_pool.shape
    plan = backend.decode_plan(c.tables, c.lens, c.block_size, c.q.shape[1], Hkv, d, NB, c.window)
    out = backend.paged_attention(c.q, c.k_pool, c.v_pool, c.tables, c.lens, c.block_size, c.window,
                                  gate=c.gate if gate else None, plan=plan)
    torch.cuda.synchronize()
    return out.cpu()


PLAN_CASES = {
    "config3": lambda: wl.c3_paged_decode(),
    "config1": lambda: wl.c1_paged_decode(),
    "reference_lengths_bf16": lambda: wl.paged_decode_case(REF_LENS, 32, 8, 2, 256, 16, torch.bfloat16, seed=21),
    "reference_lengths_fp32_14_2_64": lambda: wl.paged_decode_case(REF_LENS, 32, 14, 2, 64, 16, seed=22),
    "group8_16_2_128": lambda: wl.paged_decode_case([5, 900, 77, 3000], 400, 16, 2, 128, 16, torch.bfloat16,
                                                    seed=23),
    "block_size_4": lambda: wl.paged_decode_case(REF_LENS + [700], 300, 8, 2, 256, 4, torch.bfloat16, seed=24),
    "block_size_32": lambda: wl.paged_decode_case(REF_LENS + [4000], 300, 16, 4, 128, 32, torch.bfloat16, seed=25),
    "window_128": lambda: wl.paged_decode_case([3, 130, 700, 5000], 500, 8, 2, 256, 16, torch.bfloat16, seed=26,
                                               window=128),
    "by_cost_with_empty": lambda: wl.paged_decode_case(
        [0, 9000, 1, 0, 7000, 17, 0, 12000, 300, 0, 9000, 16, 8192, 0, 2, 11000, 33, 0, 9500, 5], 6000, 8, 2, 256,
        16, torch.bfloat16, seed=27),
    "batch_300": lambda: wl.paged_decode_case([(37 * i) % 2500 + 1 for i in range(300)], 50000, 8, 2, 256, 16,
                                              torch.bfloat16, seed=28),
}


@pytest.mark.parametrize("name", list(PLAN_CASES))
def test_plan_gives_the_same_bits(backend, name):
    """rk_paged_decode_planned reads the partition, the ranges and each group's first tiles from the plan instead of
    deriving them: the same partition and arithmetic, so bit-identical outputs, over both split instances (8-wave
    config 3, 4-wave small grids), the group-8 instance, unaligned and larger blocks, a window, ranges cut by cost
    with empty sequences, and a batch past 64 sequences (per-sequence arrays past one wave's lanes). The workspace
    is NaN-filled first."""
    from native import kernels
    case = PLAN_CASES[name]()
    want = gpu(backend, case, gate=True)
    NB, bs, Hkv, d = case.k_pool.shape
    need = backend.lib.lib.rk_paged_decode_workspace_bytes(case.q.shape[0], case.q.shape[1], Hkv, d, bs,
                                                           case.tables.shape[1])
    kernels.workspace(torch.device(DEV), need).view(torch.float32).fill_(float("nan"))
    got = planned(backend, case, gate=True)
    assert torch.equal(got, want), name


def test_plan_shared_by_layers_and_refused_for_another_layout(backend):
    """One plan serves several layers' pools with the same tables and lengths (each layer's bits equal its own
    unplanned call); a plan made for other tables is refused on the host."""
    from native import kernels
    case = wl.c3_paged_decode()
    c = case.to(DEV)
    NB, bs, Hkv, d = c.k_pool.shape
    plan = backend.decode_plan(c.tables, c.lens, bs, 8, Hkv, d, NB)
    g = torch.Generator().manual_seed(29)
    for layer in range(3):
        kp = (torch.randn(c.k_pool.shape, generator=g) * (layer + 1)).to(torch.bfloat16).to(DEV)
        vp = torch.randn(c.v_pool.shape, generator=g).to(torch.bfloat16).to(DEV)
        a = backend.paged_attention(c.q, kp, vp, c.tables, c.lens, bs, gate=c.gate, plan=plan)
        b = backend.paged_attention(c.q, kp, vp, c.tables, c.lens, bs, gate=c.gate)
        assert torch.equal(a, b), f"layer {layer}"
    other = c.tables.clone()
    with pytest.raises(ValueError):
        backend.paged_attention(c.q, c.k_pool, c.v_pool, other, c.lens, bs, plan=plan)
