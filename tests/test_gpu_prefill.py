"""P4 parity: the packed prefill attention kernel (rk_paged_prefill) vs the CPU oracle (oracle/prefill_ref.py, the
reference's per-segment write -> read -> causal attention -> gate).

The kernel's products run on bf16 MFMA operands (q, k, v as stored; probabilities rounded to bf16) with fp32
accumulation, so outputs are held to the north-star bar for bf16 outputs: within 1e-2 relative (max|diff| /
max|ref|) of the fp32 oracle. The KV write-back is a copy (with fp32 -> bf16 rounding to nearest even) and must leave
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


def run_gpu(backend, case, gate=True):
    c = case.to(DEV)
    out = backend.paged_prefill_attention(c.q, c.k_new, c.v_new, c.k_pool, c.v_pool, c.tables, c.cu_seqlens,
                                          c.starts, c.block_size, gate=c.gate if gate else None)
    torch.cuda.synchronize()
    return out.cpu(), c.k_pool.cpu(), c.v_pool.cpu()


def run_oracle(case, gate=True):
    c = case.clone()
    out = prefill_ref.packed_prefill(c.q, c.k_new, c.v_new, c.k_pool, c.v_pool, c.tables, c.cu_seqlens, c.starts,
                                     c.block_size, c.gate if gate else None)
    return out, c.k_pool, c.v_pool


@pytest.mark.parametrize("Hq,Hkv,d", [(8, 2, 256), (16, 4, 128)])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_small_segments(backend, Hq, Hkv, d, dtype):
    case = wl.prefill_case([5, 40, 100, 1, 33], [0, 17, 64, 200, 31], Hq, Hkv, d, 16, dtype, seed=7)
    got, gk, gv = run_gpu(backend, case)
    want, wk, wv = run_oracle(case)
    err = rel_err(got, want)
    print(f"prefill {Hq}/{Hkv} x {d} {dtype}: rel err {err:.2e}")
    assert torch.isfinite(got).all() and err < 1e-2
    assert torch.equal(gk, wk) and torch.equal(gv, wv)


def test_packed_equals_segment_by_segment(backend):
    case = wl.prefill_case([70, 129, 3], [50, 0, 500], seed=8)
    packed, _, _ = run_gpu(backend, case)
    for s in range(3):
        lo, hi = case.cu_seqlens[s], case.cu_seqlens[s + 1]
        one = wl.PrefillCase(case.q[lo:hi], case.k_new[lo:hi], case.v_new[lo:hi], case.gate[lo:hi], case.k_pool,
                             case.v_pool, case.tables[s:s + 1], [0, hi - lo], [case.starts[s]], case.block_size)
        alone, _, _ = run_gpu(backend, one)
        assert torch.equal(alone, packed[lo:hi])


def test_block_size_32_and_no_gate(backend):
    case = wl.prefill_case([64, 65, 17], [96, 3, 0], block_size=32, seed=9)
    got, _, _ = run_gpu(backend, case, gate=False)
    want, _, _ = run_oracle(case, gate=False)
    assert rel_err(got, want) < 1e-2


def test_config5_full_size(backend):
    case = wl.c5_prefill()
    got, gk, gv = run_gpu(backend, case)
    want, wk, wv = run_oracle(case)
    err = rel_err(got, want)
    print(f"config 5: {case.q.shape[0]} new tokens over prefixes {case.starts}: rel err {err:.2e}")
    assert torch.isfinite(got).all() and err < 1e-2
    assert torch.equal(gk, wk) and torch.equal(gv, wv)


def test_split_blocks(backend, monkeypatch):
    """Blocks whose key range is cut into pieces (here every 2 tiles, so up to ~30 pieces per block): within the bar
    of the oracle, equal across two calls (the pieces are combined in piece order whatever finishes last), and a
    packed call gives the bits of each segment alone (the cuts depend only on the block). The arrival counters are
    left at zero."""
    from native import kernels
    case = wl.prefill_case([70, 129, 3, 40], [50, 900, 500, 0], seed=11)
    want, wk, wv = run_oracle(case)
    monkeypatch.setattr(kernels, "PREFILL_SPLIT_TILES", 2)
    got, gk, gv = run_gpu(backend, case)
    again, _, _ = run_gpu(backend, case)
    assert torch.isfinite(got).all() and rel_err(got, want) < 1e-2
    assert torch.equal(got, again)
    assert torch.equal(gk, wk) and torch.equal(gv, wv)
    for s in range(4):
        lo, hi = case.cu_seqlens[s], case.cu_seqlens[s + 1]
        one = wl.PrefillCase(case.q[lo:hi], case.k_new[lo:hi], case.v_new[lo:hi], case.gate[lo:hi], case.k_pool,
                             case.v_pool, case.tables[s:s + 1], [0, hi - lo], [case.starts[s]], case.block_size)
        alone, _, _ = run_gpu(backend, one)
        assert torch.equal(alone, got[lo:hi])
    assert int(kernels.linear_counters(torch.device(DEV), 1).abs().sum()) == 0


def test_auto_split_long_prefix(backend):
    """One chunk over a long prefix, the case the automatic split is for: 3 blocks x 2 KV heads would leave most
    CUs idle, so each block is cut into pieces of at least the minimum size; within the bar of the oracle and equal
    across two calls."""
    from native import kernels
    case = wl.prefill_case([96], [12000], seed=13)
    _, n_slots = kernels.prefill_work([96], [12000], None, True, None, 2, kernels.device_cus(torch.device(DEV)))
    assert n_slots > 3
    want, wk, wv = run_oracle(case)
    got, gk, gv = run_gpu(backend, case)
    again, _, _ = run_gpu(backend, case)
    err = rel_err(got, want)
    print(f"96 queries after 12000 keys, {n_slots} pieces: rel err {err:.2e}")
    assert torch.isfinite(got).all() and err < 1e-2
    assert torch.equal(got, again)
    assert torch.equal(gk, wk) and torch.equal(gv, wv)
    assert int(kernels.linear_counters(torch.device(DEV), 1).abs().sum()) == 0


def test_bad_group_size_refused(backend):
    """Group sizes other than 4 have no kernel instance: the wrapper refuses before launching, and so does the C
    entry point if called directly."""
    case = wl.prefill_case([8], [0], 8, 1, 128, seed=10).to(DEV)
    with pytest.raises(NotImplementedError):
        backend.paged_prefill_attention(case.q, case.k_new, case.v_new, case.k_pool, case.v_pool, case.tables,
                                        case.cu_seqlens, case.starts, 16)
    from native.rocm_native import RocmKernelError
    meta = torch.tensor([0, 8, 0, 0, 0, 1, -1, 1], dtype=torch.int32, device=DEV)
    out = torch.empty(8, 8, 128, device=DEV)
    with pytest.raises(RocmKernelError):
        backend.lib.call("rk_paged_prefill", out.data_ptr(), case.q.data_ptr(), 1, case.k_new.data_ptr(),
                         case.v_new.data_ptr(), 1, case.k_pool.data_ptr(), case.v_pool.data_ptr(), 1,
                         case.tables.data_ptr(), case.tables.shape[1], meta.data_ptr(), meta.data_ptr() + 8,
                         meta.data_ptr() + 12, 1, 1, 8, 8, 1, 128, 16, case.k_pool.shape[0], None, 0, 0, 1,
                         0, None, 0, None, None)
