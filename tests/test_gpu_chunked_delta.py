"""P3 parity: the chunked gated delta rule kernels (rk_gated_delta_chunked) vs the CPU oracle's restatement of
ops.gated_delta_chunked (oracle/ops_ref.py, pinned against float64 brute force and transformers' routines) and the
float64 fixture at the kernel's shape (tests/golden/delta_rule_128.npz).

Outputs and final states are fp32 results, held to the fp32 bar: within 1e-5 relative (max|diff| / max|ref|). The
kernel's contractions with an fp32 operand use exact three-piece bf16 splits on MFMA, so this bar holds for both
input paths (bf16 inputs, as config 4 stores them, and fp32 inputs, as the model passes them). Packing several
sequences into one launch must give bit-identical rows and states to launching each alone.
"""
import numpy as np
import pytest
import torch

import workloads as wl
from helpers import rel_err
from oracle import ops_ref

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
TOL = 1e-5
GOLD = __import__("pathlib").Path(__file__).resolve().parent / "golden"


def oracle_run(case):
    outs, states = [], []
    for i, (lo, hi) in enumerate(zip(case.cu_seqlens, case.cu_seqlens[1:])):
        if hi == lo:
            states.append(case.S[i].clone())
            continue
        f = lambda x: x[lo:hi].float()
        o, S = ops_ref.gated_delta_chunked(f(case.q), f(case.k), f(case.v), f(case.beta), f(case.g), case.S[i].clone())
        outs.append(o)
        states.append(S)
    return torch.cat(outs), torch.stack(states)


def gpu_run(backend, case, dtype=None):
    c = case.to(DEV)
    cast = (lambda x: x.to(dtype)) if dtype is not None else (lambda x: x)
    S = c.S.clone()
    o = backend.gated_delta_packed(cast(c.q), cast(c.k), cast(c.v), c.beta, c.g, c.cu_seqlens, S)
    torch.cuda.synchronize()
    return o.cpu(), S.cpu()


def test_fixture_at_kernel_shape(backend):
    f = np.load(GOLD / "delta_rule_128.npz")
    wide = lambda b: torch.from_numpy((b.astype(np.uint32) << 16).view(np.float32))
    q, k, v, S0 = (wide(f[n]) for n in ("q_bf16", "k_bf16", "v_bf16", "S0_bf16"))
    beta, g = torch.from_numpy(f["beta"]), torch.from_numpy(f["g"])
    for dtype in (torch.bfloat16, torch.float32):
        args = [x.to(DEV, dtype) for x in (q, k, v)] + [beta.to(DEV), g.to(DEV), S0.to(DEV)]
        o, S = backend.gated_delta(*args)
        torch.cuda.synchronize()
        eo, es = rel_err(o.cpu(), f["out"]), rel_err(S.cpu(), f["S"])
        print(f"fixture {dtype}: out {eo:.2e}, state {es:.2e}")
        assert eo < TOL and es < TOL
        assert torch.equal(S0, args[-1].cpu())           # gated_delta leaves its input state alone


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_packed_lengths_match_oracle(backend, dtype):
    case = wl.chunked_delta_case([1, 5, 64, 65, 130, 200], H=4, dtype=dtype, seed=11, state_scale=0.1)
    o, S = gpu_run(backend, case)
    wo, ws = oracle_run(case)
    eo, es = rel_err(o, wo), rel_err(S, ws)
    print(f"lengths 1..200 {dtype}: out {eo:.2e}, state {es:.2e}")
    assert torch.isfinite(o).all() and eo < TOL and es < TOL


def test_packed_equals_per_sequence(backend):
    case = wl.chunked_delta_case([70, 3, 129], H=2, seed=12, state_scale=0.1)
    o, S = gpu_run(backend, case)
    for i, (lo, hi) in enumerate(zip(case.cu_seqlens, case.cu_seqlens[1:])):
        one = wl.ChunkedDeltaCase(case.q[lo:hi], case.k[lo:hi], case.v[lo:hi], case.beta[lo:hi], case.g[lo:hi],
                                  case.S[i:i + 1], [0, hi - lo])
        oi, Si = gpu_run(backend, one)
        assert torch.equal(oi, o[lo:hi]) and torch.equal(Si[0], S[i])


def test_empty_sequences_in_a_pack(backend):
    case = wl.chunked_delta_case([0, 70, 0, 3], H=2, seed=13, state_scale=0.1)
    o, S = gpu_run(backend, case)
    wo, ws = oracle_run(case)
    assert torch.equal(S[0], case.S[0]) and torch.equal(S[2], case.S[2])
    assert rel_err(o, wo) < TOL and rel_err(S, ws) < TOL


def test_zero_beta_and_decay_leave_state_unchanged(backend):
    case = wl.chunked_delta_case([100], H=2, seed=14, state_scale=0.1)
    case.beta.zero_()
    case.g.zero_()
    o, S = gpu_run(backend, case)
    wo, _ = oracle_run(case)
    assert torch.equal(S, case.S)                         # e^0 S + K^T 0, exactly
    assert rel_err(o, wo) < TOL                           # o = Q S


def test_single_token_equals_recurrent(backend):
    case = wl.chunked_delta_case([1], H=4, dtype=torch.float32, seed=15, state_scale=0.1)
    c = case.to(DEV)
    o, S = backend.gated_delta(c.q, c.k, c.v, c.beta, c.g, c.S[0])
    wo, ws = ops_ref.gated_delta_recurrent(case.q, case.k, case.v, case.beta, case.g, case.S[0].clone())
    assert rel_err(o.cpu(), wo) < TOL and rel_err(S.cpu(), ws) < TOL


def test_pool_states_through_seq_index(backend):
    """States of a HybridPool-shaped array [seqs, n_linear, H, dk, dv]: one layer slot viewed with a stride, sequences
    mapped to pool rows by seq_index; other rows and the other layer slot stay untouched."""
    case = wl.chunked_delta_case([90, 33, 64], H=2, seed=16, state_scale=0.1)
    pool = torch.randn(5, 2, 2, 128, 128, generator=torch.Generator().manual_seed(17)) * 0.1
    idx = [3, 0, 4]
    for i, j in enumerate(idx):
        pool[j, 1] = case.S[i]
    pool_d = pool.to(DEV)
    c = case.to(DEV)
    o = backend.gated_delta_packed(c.q, c.k, c.v, c.beta, c.g, c.cu_seqlens, pool_d[:, 1],
                                   torch.tensor(idx, dtype=torch.int32, device=DEV))
    torch.cuda.synchronize()
    got = pool_d.cpu()
    wo, ws = oracle_run(case)
    assert rel_err(o.cpu(), wo) < TOL
    for i, j in enumerate(idx):
        assert rel_err(got[j, 1], ws[i]) < TOL
    assert torch.equal(got[:, 0], pool[:, 0]) and torch.equal(got[[1, 2], 1], pool[[1, 2], 1])


def test_config4_full_size(backend):
    case = wl.c4_chunked_delta()
    o, S = gpu_run(backend, case)
    wo, ws = oracle_run(case)
    eo, es = rel_err(o, wo), rel_err(S, ws)
    print(f"config 4: 4 x 4096 tokens, 16 heads: out {eo:.2e}, state {es:.2e}")
    assert torch.isfinite(o).all() and eo < TOL and es < TOL


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_many_short_ragged_sequences(backend, dtype):
    """40 sequences of 0 .. 150 tokens (single-chunk and partial-chunk sequences everywhere, empty ones between):
    the bf16 scan's loading waves repeat a short chunk's last K / Q / V row and compute P from those rows."""
    lens = [int(x) for x in np.random.default_rng(21).integers(0, 151, size=40)]
    lens[3] = lens[17] = 0
    lens[5], lens[6] = 1, 64
    case = wl.chunked_delta_case(lens, H=2, dtype=dtype, seed=22, state_scale=0.1)
    o, S = gpu_run(backend, case)
    wo, ws = oracle_run(case)
    eo, es = rel_err(o, wo), rel_err(S, ws)
    print(f"40 ragged sequences {dtype}: out {eo:.2e}, state {es:.2e}")
    assert torch.isfinite(o).all() and eo < TOL and es < TOL
    assert torch.equal(S[3], case.S[3]) and torch.equal(S[17], case.S[17])


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_workspace_needs_no_clearing(backend, dtype):
    """The per-chunk workspace is written in full by the prep before the scan reads it: a workspace holding NaN
    bytes and one holding zeros give the same bits."""
    from native import kernels
    case = wl.chunked_delta_case([70, 129, 1, 64], H=4, dtype=dtype, seed=23, state_scale=0.1)
    runs = []
    for fill in (0xFF, 0x00):
        kernels.workspace(torch.device(DEV), 16 << 20).fill_(fill)   # the buffer the launch reuses (> its need)
        runs.append(gpu_run(backend, case))
    assert torch.equal(runs[0][0], runs[1][0]) and torch.equal(runs[0][1], runs[1][1])
    assert torch.isfinite(runs[0][0]).all()
