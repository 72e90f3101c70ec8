"""P2 parity: the fused HIP DeltaNet decode step (rk_deltanet_decode) vs the CPU oracle
(TorchBackend.deltanet_decode_batch restated), on BASELINE config 2 and on the reference's 4-step carried test
(tests/test_qwen35.py:101-122: slot 1 of 3, conv_w = 0.5 N, A_log, dt_bias ~ N, a = 3 N, norm_w = 1 + 0.1 N).

Bars: output and state within 1e-5 relative (max|diff| / max|ref|) per step; the conv tail is a copy of raw inputs,
so it must match exactly; slots outside the batch must be untouched (torch.equal).
"""
import pytest
import torch

import workloads as wl
from helpers import SlotState, rel_err
from oracle import backend_ref

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def oracle_step(case):
    """Run the oracle on CPU copies of the pool slots the batch uses; returns (out, S, conv) pool tensors."""
    S, conv = case.S.clone(), case.conv.clone()
    states = [SlotState(S[int(s)], conv[int(s)]) for s in case.seq_index]
    out = backend_ref.deltanet_decode_batch(case.qkv, case.z, case.b, case.a, states, case.slot, case.conv_w,
                                            case.A_log, case.dt_bias, case.norm_w, case.eps, case.dims)
    return out, S, conv


def gpu_step(backend, case):
    from native import kernels
    c = case.to(DEV)
    out = kernels.deltanet_decode(c.qkv, c.z, c.b, c.a, c.conv, c.S, c.seq_index, c.slot, c.conv_w, c.A_log,
                                  c.dt_bias, c.norm_w, c.eps, c.dims)
    torch.cuda.synchronize()
    return out.cpu(), c.S.cpu(), c.conv.cpu()


def test_config2(backend):
    case = wl.c2_deltanet_step(max_seqs=12, n_linear=3, slot=1)
    want_out, want_S, want_conv = oracle_step(case)
    got_out, got_S, got_conv = gpu_step(backend, case)
    e_out, e_S = rel_err(got_out, want_out), rel_err(got_S, want_S)
    print(f"config 2: out rel {e_out:.2e}, state rel {e_S:.2e}")
    assert e_out < 1e-5 and e_S < 1e-5
    assert torch.equal(got_conv, want_conv)
    untouched = [i for i in range(12) if i not in case.seq_index.tolist()]
    assert torch.equal(got_S[untouched], case.S[untouched]) and torch.equal(got_conv[untouched], case.conv[untouched])
    assert torch.equal(got_S[:, [0, 2]], case.S[:, [0, 2]])          # other layers of the used slots


def test_four_carried_steps_through_backend(backend):
    """The reference's fused-kernel test, through RocmBackend.deltanet_decode with a standalone state."""
    H, dk, dv, KD, C = 16, 128, 128, 2048, 6144
    gen = torch.Generator().manual_seed(0)
    r = lambda *s, scale=1.0: torch.randn(*s, generator=gen) * scale
    conv_w, A_log, dt_bias, norm_w = r(C, 4, scale=0.5), r(H), r(H), 1 + r(dv, scale=0.1)
    tail, S = r(3, 3, C), r(3, H, dk, dv, scale=0.05)
    ref = SlotState(S.clone(), tail.clone())
    dev = SlotState(S.clone().to(DEV), tail.clone().to(DEV))
    dev.pool = None
    worst = 0.0
    for step in range(4):
        qkv, z, bl, a = r(1, C), r(1, H * dv), r(1, H), r(1, H, scale=3)
        o_ref = backend_ref.deltanet_decode(qkv, z, bl, a, ref, 1, conv_w, A_log, dt_bias, norm_w, 1e-6,
                                            (H, dk, dv, KD))
        o_dev = backend.deltanet_decode(qkv.to(DEV), z.to(DEV), bl.to(DEV), a.to(DEV), dev, 1, conv_w.to(DEV),
                                        A_log.to(DEV), dt_bias.to(DEV), norm_w.to(DEV), 1e-6, (H, dk, dv, KD))
        worst = max(worst, rel_err(o_dev, o_ref), rel_err(dev.S, ref.S))
        assert torch.equal(dev.conv_tail.cpu(), ref.conv_tail)
    print(f"4 carried steps: worst rel {worst:.2e}")
    assert worst < 1e-5
    assert torch.equal(dev.S[0].cpu(), S[0]) and torch.equal(dev.S[2].cpu(), S[2])


def test_pool_states_one_launch(backend):
    """States of one HybridPool decode together; mixed standalone states run one by one; both match the oracle."""
    gen = torch.Generator().manual_seed(5)
    H, dk, dv, KD, C = 16, 128, 128, 2048, 6144
    pool = wl.StateSlots(4, 2, H, dk, dv, C, 4, device=DEV)
    states = pool.views(range(3))
    pool.S.normal_(0, 0.02, generator=torch.Generator(device=DEV).manual_seed(1))
    pool.conv.normal_(0, 1, generator=torch.Generator(device=DEV).manual_seed(2))
    refs = [SlotState(st.S.cpu().clone(), st.conv_tail.cpu().clone()) for st in states]
    r = lambda *s, scale=1.0: torch.randn(*s, generator=gen) * scale
    conv_w, A_log, dt_bias, norm_w = r(C, 4, scale=0.5), r(H), r(H), 1 + r(dv, scale=0.1)
    qkv, z, bl, a = r(3, C), r(3, H * dv), r(3, H), r(3, H)
    want = backend_ref.deltanet_decode_batch(qkv, z, bl, a, refs, 1, conv_w, A_log, dt_bias, norm_w, 1e-6,
                                             (H, dk, dv, KD))
    got = backend.deltanet_decode_batch(qkv.to(DEV), z.to(DEV), bl.to(DEV), a.to(DEV), states, 1, conv_w.to(DEV),
                                        A_log.to(DEV), dt_bias.to(DEV), norm_w.to(DEV), 1e-6, (H, dk, dv, KD))
    assert rel_err(got, want) < 1e-5
    for st, rf in zip(states, refs):
        assert rel_err(st.S, rf.S) < 1e-5
        assert torch.equal(st.conv_tail.cpu(), rf.conv_tail)





def test_batch_sizes_back_to_back(backend):
    """Calls of different batch sizes back to back on one pool (rows 0 .. B-1 of a 10-row pool) each match the
    oracle and touch only their own rows."""
    for batch in (8, 3, 8):
        case = wl.c2_deltanet_step(seed=40 + batch, batch=batch, max_seqs=10)
        want_out, want_S, want_conv = oracle_step(case)
        got_out, got_S, got_conv = gpu_step(backend, case)
        assert rel_err(got_out, want_out) < 1e-5 and rel_err(got_S, want_S) < 1e-5
        assert torch.equal(got_conv, want_conv)
