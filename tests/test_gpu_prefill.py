"""P4 parity: the packed prefill attention kernel (rk_paged_prefill) vs the CPU oracle (oracle/prefill_ref.py, the
reference's per-segment write -> read -> causal attention -> gate).

The reference computes in fp32 on widened inputs (src/ops.py:84-87). bf16 q and pool run on bf16 MFMA operands
(probabilities rounded to bf16) with fp32 accumulation: 32 queries per wave at 4 query heads per kv-head (config 5),
16 queries per wave for every other group size, head_dim 64 and block size 1; they are held to the bar for bf16
outputs, 1e-2 relative (max|diff| / max|ref|) of the fp32 oracle. fp32 inputs (the Qwen3.5 engine's own fp32 pools,
src/models/qwen3_5.py:70-71) and exact=True run on fp32 operands and are held to 1e-5. The KV write-back is a copy (with fp32 -> bf16 rounding to nearest even) and must leave
the pool bit-identical to the oracle's; packing segments together must give bit-identical rows to running each
segment alone under one split size (a block's cuts depend only on the block; the automatic size depends on the
whole batch, so under it a segment alone may be cut where the packed batch is not).
"""
import pytest
import torch

import workloads as wl
from helpers import rel_err
from oracle import prefill_ref

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


TOL_F32 = 1e-5
TOL_BF16 = 1e-2


def run_gpu(backend, case, gate=True, exact=False):
    c = case.to(DEV)
    out = backend.paged_prefill_attention(c.q, c.k_new, c.v_new, c.k_pool, c.v_pool, c.tables, c.cu_seqlens,
                                          c.starts, c.block_size, gate=c.gate if gate else None, exact=exact)
    torch.cuda.synchronize()
    return out.cpu(), c.k_pool.cpu(), c.v_pool.cpu()


def run_oracle(case, gate=True):
    c = case.clone()
    out = prefill_ref.packed_prefill(c.q, c.k_new, c.v_new, c.k_pool, c.v_pool, c.tables, c.cu_seqlens, c.starts,
                                     c.block_size, c.gate if gate else None)
    return out, c.k_pool, c.v_pool


@pytest.mark.parametrize("Hq,Hkv,d", [(8, 2, 256), (16, 4, 128), (14, 2, 64), (8, 8, 128), (16, 2, 256)])
@pytest.mark.parametrize("dtype,exact,tol", [(torch.bfloat16, False, TOL_BF16), (torch.bfloat16, True, TOL_F32),
                                             (torch.float32, False, TOL_F32)])
def test_small_segments(backend, Hq, Hkv, d, dtype, exact, tol):
    case = wl.prefill_case([5, 40, 100, 1, 33], [0, 17, 64, 200, 31], Hq, Hkv, d, 16, dtype, seed=7)
    got, gk, gv = run_gpu(backend, case, exact=exact)
    want, wk, wv = run_oracle(case)
    err = rel_err(got, want)
    print(f"prefill {Hq}/{Hkv} x {d} {dtype} exact {exact}: rel err {err:.2e}")
    assert torch.isfinite(got).all() and err < tol
    assert torch.equal(gk, wk) and torch.equal(gv, wv)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_packed_equals_segment_by_segment(backend, dtype):
    case = wl.prefill_case([70, 129, 3], [50, 0, 500], dtype=dtype, seed=8)
    packed, _, _ = run_gpu(backend, case)
    for s in range(3):
        lo, hi = case.cu_seqlens[s], case.cu_seqlens[s + 1]
        one = wl.PrefillCase(case.q[lo:hi], case.k_new[lo:hi], case.v_new[lo:hi], case.gate[lo:hi], case.k_pool,
                             case.v_pool, case.tables[s:s + 1], [0, hi - lo], [case.starts[s]], case.block_size)
        alone, _, _ = run_gpu(backend, one)
        assert torch.equal(alone, packed[lo:hi])


@pytest.mark.parametrize("dtype,exact,tol", [(torch.bfloat16, False, TOL_BF16), (torch.bfloat16, True, TOL_F32),
                                             (torch.float32, False, TOL_F32)])
@pytest.mark.parametrize("bs", [32, 1, 5])
def test_block_sizes_and_no_gate(backend, dtype, exact, tol, bs):
    """Block sizes 32, 5 and 1 (a bf16 pool of one-position blocks runs on the 16-query bf16 kernel)."""
    case = wl.prefill_case([64, 65, 17], [96, 3, 0], block_size=bs, dtype=dtype, seed=9)
    got, _, _ = run_gpu(backend, case, gate=False, exact=exact)
    want, _, _ = run_oracle(case, gate=False)
    assert rel_err(got, want) < tol


@pytest.mark.parametrize("dtype,exact,tol", [(torch.bfloat16, False, TOL_BF16), (torch.bfloat16, True, TOL_F32),
                                             (torch.float32, False, TOL_F32)])
def test_config5_full_size(backend, dtype, exact, tol):
    """Config 5 as specified (bf16, on bf16 operands), the same batch with exact=True, and with the engine's fp32
    pool (src/models/qwen3_5.py:70-71)."""
    case = wl.c5_prefill(dtype=dtype)
    got, gk, gv = run_gpu(backend, case, exact=exact)
    want, wk, wv = run_oracle(case)
    err = rel_err(got, want)
    print(f"config 5 {dtype} exact {exact}: {case.q.shape[0]} new tokens over prefixes {case.starts}: rel err "
          f"{err:.2e}")
    assert torch.isfinite(got).all() and err < tol
    assert torch.equal(gk, wk) and torch.equal(gv, wv)


@pytest.mark.parametrize("dtype,Hq,Hkv,d,tol", [(torch.bfloat16, 8, 2, 256, TOL_BF16), (torch.float32, 8, 2, 256, TOL_F32),
                                                (torch.bfloat16, 14, 2, 64, TOL_BF16), (torch.float32, 14, 2, 64, TOL_F32)])
def test_split_blocks(backend, monkeypatch, dtype, Hq, Hkv, d, tol):
    """Blocks whose key range is cut into pieces (here every 2 tiles, so up to ~30 pieces per block): within the bar
    of the oracle, equal across two calls (the pieces are combined in piece order whatever finishes last), and a
    packed call gives the bits of each segment alone (the cuts depend only on the block). The arrival counters are
    left at zero. All three kernels: bf16 operands on 32 and on 16 queries per wave (a group of 7 over two head
    chunks), fp32 operands (fp32 pool)."""
    from native import kernels
    case = wl.prefill_case([70, 129, 3, 40], [50, 900, 500, 0], Hq, Hkv, d, dtype=dtype, seed=11)
    want, wk, wv = run_oracle(case)
    monkeypatch.setattr(kernels, "PREFILL_SPLIT_TILES", 2)
    got, gk, gv = run_gpu(backend, case)
    again, _, _ = run_gpu(backend, case)
    err = rel_err(got, want)
    print(f"split blocks {dtype} {Hq}/{Hkv}x{d}: rel err {err:.2e}")
    assert torch.isfinite(got).all() and err < tol
    assert torch.equal(got, again)
    assert torch.equal(gk, wk) and torch.equal(gv, wv)
    for s in range(4):
        lo, hi = case.cu_seqlens[s], case.cu_seqlens[s + 1]
        one = wl.PrefillCase(case.q[lo:hi], case.k_new[lo:hi], case.v_new[lo:hi], case.gate[lo:hi], case.k_pool,
                             case.v_pool, case.tables[s:s + 1], [0, hi - lo], [case.starts[s]], case.block_size)
        alone, _, _ = run_gpu(backend, one)
        assert torch.equal(alone, got[lo:hi])
    assert int(kernels.linear_counters(torch.device(DEV), 1).abs().sum()) == 0


@pytest.mark.parametrize("dtype,tol", [(torch.bfloat16, TOL_BF16), (torch.float32, TOL_F32)])
def test_auto_split_long_prefix(backend, dtype, tol):
    """One chunk over a long prefix, the case the automatic split is for: 3 blocks x 2 KV heads would leave most
    CUs idle, so each block is cut into pieces of at least the minimum size; within the bar of the oracle and equal
    across two calls."""
    from native import kernels
    case = wl.prefill_case([96], [12000], dtype=dtype, seed=13)
    _, n_slots = kernels.prefill_work([96], [12000], None, True, None, 2, kernels.device_cus(torch.device(DEV)))
    assert n_slots > 3
    want, wk, wv = run_oracle(case)
    got, gk, gv = run_gpu(backend, case)
    again, _, _ = run_gpu(backend, case)
    err = rel_err(got, want)
    print(f"96 queries after 12000 keys {dtype}, {n_slots} pieces: rel err {err:.2e}")
    assert torch.isfinite(got).all() and err < tol
    assert torch.equal(got, again)
    assert torch.equal(gk, wk) and torch.equal(gv, wv)
    assert int(kernels.linear_counters(torch.device(DEV), 1).abs().sum()) == 0


def test_unsupported_head_dim_refused(backend):
    """head_dim 96 has no kernel instance: the wrapper refuses before launching, and so does the C entry point if
    called directly (RK_ERR_UNSUPPORTED)."""
    from native import kernels
    case = wl.prefill_case([8], [0], 8, 2, 96, seed=10).to(DEV)
    with pytest.raises(NotImplementedError):
        backend.paged_prefill_attention(case.q, case.k_new, case.v_new, case.k_pool, case.v_pool, case.tables,
                                        case.cu_seqlens, case.starts, 16)
    meta = torch.tensor([0, 8, 0, 0, 0, 1, -1, 1], dtype=torch.int32, device=DEV)
    out = torch.empty(8, 8, 96, device=DEV)
    rc = backend.lib.lib.rk_paged_prefill(out.data_ptr(), case.q.data_ptr(), 1, case.k_new.data_ptr(),
                                          case.v_new.data_ptr(), 1, case.k_pool.data_ptr(), case.v_pool.data_ptr(), 1,
                                          case.tables.data_ptr(), case.tables.shape[1], meta.data_ptr(),
                                          meta.data_ptr() + 8, meta.data_ptr() + 12, 1, 1, 8, 8, 2, 96, 16,
                                          case.k_pool.shape[0], None, 0, 0, 1, 0, 0, None, 0, None, 0,
                                          kernels._stream(torch.device(DEV)))
    assert rc == 2


@pytest.mark.parametrize("dtype,Hq,Hkv,d,tol", [(torch.bfloat16, 8, 2, 256, TOL_BF16), (torch.bfloat16, 14, 2, 64, TOL_BF16),
                                                (torch.float32, 8, 2, 256, TOL_F32)])
def test_split_item_with_an_empty_piece(backend, dtype, Hq, Hkv, d, tol):
    """A work list written by hand (through the C ABI) whose split block has a first piece lying wholly below the
    block's window, so that piece has no tiles: it still writes its (empty) record and counts in, and the block's
    output is the other piece's, within the bar of the oracle. All three kernels (32- and 16-query bf16 operands,
    fp32 operands)."""
    from native import kernels
    from oracle import ops_ref
    W, n, p = 40, 32, 300                          # one 32-query block at positions 300 .. 331, window 40
    case = wl.prefill_case([n], [p], Hq, Hkv, d, 16, dtype, seed=21)
    c = case.to(DEV)
    out = torch.empty(n, Hq, d, dtype=torch.float32, device=DEV)
    kmin = p - W + 1                               # the block's first visible key: tile kmin // 32 = 8
    t_lo, t_hi = kmin // 32, -(-(p + n) // 32)
    # piece 0 covers tiles [2, 8): below the window; piece 1 covers [8, t_hi)
    work = [0, 2, t_lo, 0, (0 << 16) | 2, 0, t_lo, t_hi, 0, (1 << 16) | 2]
    meta = torch.tensor(list(case.cu_seqlens) + list(case.starts) + work, dtype=torch.int32, device=DEV)
    lib = kernels.load()
    part_bytes = lib.lib.rk_paged_prefill_workspace_bytes(2, Hq, d)
    n_cnt = lib.lib.rk_paged_prefill_counters(2, Hq)
    part = torch.full((part_bytes // 4,), float("nan"), device=DEV)
    cnt = torch.zeros(n_cnt, dtype=torch.int32, device=DEV)
    code = kernels.DTYPE_CODES[dtype]
    NB, bs = c.k_pool.shape[0], c.k_pool.shape[1]
    lib.call("rk_paged_prefill", out.data_ptr(), c.q.data_ptr(), code, c.k_new.data_ptr(), c.v_new.data_ptr(), code,
             c.k_pool.data_ptr(), c.v_pool.data_ptr(), code, c.tables.data_ptr(), c.tables.shape[1], meta.data_ptr(),
             meta.data_ptr() + 4 * 2, meta.data_ptr() + 4 * 3, 2, 1, n, Hq, Hkv, d, bs, NB, None,
             kernels.DTYPE_CODES[torch.float32], W, 1, 0, 2, part.data_ptr(), part_bytes, cnt.data_ptr(), n_cnt,
             torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    ref = case.clone()
    table = ref.tables[0].long()
    pos = torch.arange(p, p + n)
    ref.k_pool[table[pos // bs], pos % bs] = ref.k_new.to(ref.k_pool.dtype)
    ref.v_pool[table[pos // bs], pos % bs] = ref.v_new.to(ref.v_pool.dtype)
    nb = -(-(p + n) // bs)
    K = ref.k_pool[table[:nb]].flatten(0, 1)[:p + n]
    V = ref.v_pool[table[:nb]].flatten(0, 1)[:p + n]
    want = ops_ref.attention(ref.q, K, V, causal=True, window=W)
    err = rel_err(out, want)
    which = kernels.prefill_kernel(dtype, dtype, Hq, Hkv, d, False, c.tables.shape[1], bs)
    print(f"empty split piece, {which} {Hq}/{Hkv}x{d}: rel err {err:.2e}")
    assert torch.isfinite(out).all() and err < tol
    assert int(cnt.abs().sum()) == 0
