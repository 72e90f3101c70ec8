"""Parity of the DeltaNet prefill companions (the linear-attention segment around P3, src/models/qwen3_5.py:136-162)
with the CPU oracle: rk_causal_conv1d vs TorchBackend.causal_conv1d (src/backend/torch_ref.py:49-50, x widened, then
src/ops.py:127-139), rk_rms_norm_gated vs
ops.rms_norm_gated (src/ops.py:120-124), rk_deltanet_prefill_front vs the segment front of qwen3_5.py:145-155 and
RocmBackend.deltanet_prefill (front + chunked delta rule + gated norm) vs the oracle's per-segment loop, whose
composition is pinned on the CPU against chained decode steps and split prefills.

Bars: fp32 results within 1e-5 relative (max|diff| / max|ref|), bf16 inputs included: TorchBackend.causal_conv1d
widens x before the conv (src/backend/torch_ref.py:49-50), so the fp32 old tail is used as stored and the new tail is
fp32; conv tails are copies of the widened raw inputs and carried old rows, and must match exactly; state slots
outside the batch and other layers' slots must be untouched. Packing segments into one launch must give bit-identical rows to running each
segment alone.
"""
import pytest
import torch

from helpers import SlotState, rel_err
from oracle import backend_ref, ops_ref
import workloads as wl

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
TOL = 1e-5
H, DK, DV, KD, C, K = 16, 128, 128, 2048, 6144, 4
DIMS = (H, DK, DV, KD)


def layer(seed):
    g_ = torch.Generator().manual_seed(seed)
    r = lambda *s, scale=1.0: scale * torch.randn(*s, generator=g_)
    return dict(conv_w=r(C, K, scale=0.5), A_log=r(H, scale=0.5), dt_bias=r(H, scale=0.5),
                norm_w=1.0 + r(DV, scale=0.1)), g_


def projection(N, dtype, g_):
    """The fused in_proj output [N, C | H*dv | H | H] (qkv, z, beta logits, a) of qwen3_5.py:128-133."""
    y = torch.randn(N, C + H * DV + 2 * H, generator=g_)
    y[:, -H:] *= 3.0                                                  # a: exercise softplus's range
    return y.to(dtype)


def cols(y):
    return y[:, :C], y[:, C:C + H * DV], y[:, -2 * H:-H], y[:, -H:]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("T", [1, 2, 3, 37, 257])
def test_causal_conv1d(backend, dtype, T):
    lw, g_ = layer(T)
    y = projection(T, dtype, g_)
    x = cols(y)[0]                                                    # strided rows, as the model passes them
    tail = torch.randn(K - 1, C, generator=g_)                        # fp32 values bf16 cannot hold
    u_ref, t_ref = backend_ref.causal_conv1d(x, tail, lw["conv_w"])
    u, t = backend.causal_conv1d(x.to(DEV), tail.to(DEV), lw["conv_w"].to(DEV))
    assert u.dtype == torch.float32 and t.dtype == torch.float32
    e = rel_err(u, u_ref)
    print(f"causal_conv1d T {T} {dtype}: rel {e:.2e}")
    assert e < TOL
    assert torch.equal(t.cpu(), t_ref)


@pytest.mark.parametrize("dv", [64, 128, 256, 512])
@pytest.mark.parametrize("zdtype", [torch.float32, torch.bfloat16])
def test_rms_norm_gated(backend, dv, zdtype):
    g_ = torch.Generator().manual_seed(dv)
    rows = 16 * 37
    x = torch.randn(rows, dv, generator=g_) * torch.rand(rows, 1, generator=g_) * 4
    z = (torch.randn(rows, dv, generator=g_) * 3).to(zdtype)
    w = 1.0 + 0.1 * torch.randn(dv, generator=g_)
    want = ops_ref.rms_norm_gated(x, z, w, 1e-6)
    got = backend.rms_norm_gated(x.to(DEV), z.to(DEV), w.to(DEV), 1e-6)
    e = rel_err(got, want)
    print(f"rms_norm_gated dv {dv} z {zdtype}: rel {e:.2e}")
    assert e < TOL


def test_rms_norm_gated_head_rows_of_a_projection(backend):
    """z given as the [N, H*dv] columns of a wider projection row (16 heads per row): same as the reshaped copy."""
    from native import kernels
    g_ = torch.Generator().manual_seed(3)
    y = projection(50, torch.bfloat16, g_).to(DEV)
    z = cols(y)[1]
    x = torch.randn(50 * H, DV, generator=g_).to(DEV)
    w = (1.0 + 0.1 * torch.randn(DV, generator=g_)).to(DEV)
    got = kernels.rms_norm_gated(x, z, w, 1e-6)
    want = kernels.rms_norm_gated(x, z.reshape(50 * H, DV), w, 1e-6)
    assert torch.equal(got, want)
    assert rel_err(got, ops_ref.rms_norm_gated(x.cpu(), z.cpu().reshape(50 * H, DV), w.cpu(), 1e-6)) < TOL


LENGTHS = [5, 0, 1, 2, 64, 130, 3]


def pool_with_states(g_, n):
    pool = wl.StateSlots(n + 3, 2, H, DK, DV, C, K, device=DEV)
    pool.S.copy_(0.05 * torch.randn(pool.S.shape, generator=g_))
    pool.conv.copy_(torch.randn(pool.conv.shape, generator=g_))
    return pool, pool.views(range(2, n + 2))                          # rows 0, 1 and n + 2: not in the batch


# the kernel streams runs of 32 packed tokens: runs that cross several (and empty) segments, and runs that start
# 1 or 2 tokens into a segment (window primed from the old tail and the segment's first rows)
@pytest.mark.parametrize("lengths", [LENGTHS, [30, 40, 1, 33], [31, 1, 64, 0], [31, 10, 20]])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_front_packed_with_state_handoff(backend, dtype, lengths):
    from native import kernels
    lw, g_ = layer(21)
    cu = [0]
    for n in lengths:
        cu.append(cu[-1] + n)
    y = projection(cu[-1], dtype, g_)
    pool, states = pool_with_states(g_, len(lengths))
    conv0 = pool.conv.cpu().clone()
    slot = 1
    qkv, _, b, a = cols(y.to(DEV))
    got = kernels.deltanet_prefill_front(qkv, b, a, pool.conv[:, slot], pool.seq_index(states), lw["conv_w"].to(DEV),
                                         lw["A_log"].to(DEV), lw["dt_bias"].to(DEV), cu, DIMS)
    conv = pool.conv.cpu()
    worst = 0.0
    for i, (lo, hi) in enumerate(zip(cu, cu[1:])):
        s = states[i].seq
        if hi == lo:
            assert torch.equal(conv[s], conv0[s])
            continue
        xq, _, xb, xa = cols(y[lo:hi])
        want = backend_ref.linear_attention_front(xq, xb, xa, conv0[s, slot], lw["conv_w"], lw["A_log"],
                                                  lw["dt_bias"], DIMS)
        for gt, wt in zip(got, want[:5]):
            worst = max(worst, rel_err(gt[lo:hi], wt))
        assert want[5].dtype == torch.float32
        assert torch.equal(conv[s, slot], want[5]), f"segment {i} tail"
        assert torch.equal(conv[s, 0], conv0[s, 0])                    # the other layer's slot
    print(f"front {dtype}: worst rel {worst:.2e}")
    assert worst < TOL
    unused = [0, 1]
    assert torch.equal(conv[unused], conv0[unused])


def test_front_without_state_reads_zero_tails(backend):
    from native import kernels
    lw, g_ = layer(22)
    cu = [0, 7, 7, 40]
    y = projection(40, torch.float32, g_)
    qkv, _, b, a = cols(y.to(DEV))
    got = kernels.deltanet_prefill_front(qkv, b, a, None, None, lw["conv_w"].to(DEV), lw["A_log"].to(DEV),
                                         lw["dt_bias"].to(DEV), cu, DIMS)
    for lo, hi in zip(cu, cu[1:]):
        if hi == lo:
            continue
        xq, _, xb, xa = cols(y[lo:hi])
        want = backend_ref.linear_attention_front(xq, xb, xa, torch.zeros(K - 1, C), lw["conv_w"], lw["A_log"],
                                                  lw["dt_bias"], DIMS)
        for gt, wt in zip(got, want[:5]):
            assert rel_err(gt[lo:hi], wt) < TOL


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_deltanet_prefill_matches_segment_loop(backend, dtype):
    """The whole packed linear-attention prefill (4 launches) vs the reference's per-segment loop, with pool states
    carried; the one-token segment takes the reference's decode step on the oracle side."""
    lw, g_ = layer(23)
    cu = [0]
    for n in LENGTHS:
        cu.append(cu[-1] + n)
    y = projection(cu[-1], dtype, g_)
    pool, states = pool_with_states(g_, len(LENGTHS))
    S0, conv0 = pool.S.cpu().clone(), pool.conv.cpu().clone()
    slot = 0
    ref_states = [SlotState(S0[st.seq].clone(), conv0[st.seq].clone()) for st in states]
    want = backend_ref.linear_attention_segments(*cols(y), ref_states, slot, cu, lw["conv_w"], lw["A_log"],
                                                 lw["dt_bias"], lw["norm_w"], 1e-6, DIMS)
    qkv, z, b, a = cols(y.to(DEV))
    got = backend.deltanet_prefill(qkv, z, b, a, states, slot, cu, lw["conv_w"].to(DEV), lw["A_log"].to(DEV),
                                   lw["dt_bias"].to(DEV), lw["norm_w"].to(DEV), 1e-6, DIMS)
    torch.cuda.synchronize()
    S, conv = pool.S.cpu(), pool.conv.cpu()
    e_out = rel_err(got, want)
    e_S = max(rel_err(S[st.seq, slot], rs.S[slot]) for st, rs in zip(states, ref_states))
    print(f"deltanet_prefill {dtype}: out rel {e_out:.2e}, state rel {e_S:.2e}")
    assert e_out < TOL and e_S < TOL
    for st, rs in zip(states, ref_states):
        assert torch.equal(conv[st.seq, slot], rs.conv_tail[slot])
        assert torch.equal(S[st.seq, 1], S0[st.seq, 1]) and torch.equal(conv[st.seq, 1], conv0[st.seq, 1])
    assert torch.equal(S[:2], S0[:2]) and torch.equal(conv[:2], conv0[:2])


def test_deltanet_prefill_without_state(backend):
    lw, g_ = layer(24)
    cu = [0, 70, 71, 200]
    y = projection(200, torch.float32, g_)
    want = backend_ref.linear_attention_segments(*cols(y), None, 0, cu, lw["conv_w"], lw["A_log"], lw["dt_bias"],
                                                 lw["norm_w"], 1e-6, DIMS)
    got = backend.deltanet_prefill(*cols(y.to(DEV)), None, 0, cu, lw["conv_w"].to(DEV), lw["A_log"].to(DEV),
                                   lw["dt_bias"].to(DEV), lw["norm_w"].to(DEV), 1e-6, DIMS)
    e = rel_err(got, want)
    print(f"deltanet_prefill without state: rel {e:.2e}")
    assert e < TOL


def test_packing_is_bit_identical_to_single_segments(backend):
    lw, g_ = layer(25)
    cu = [0, 100, 100, 163, 300]
    y = projection(300, torch.bfloat16, g_).to(DEV)
    args = (lw["conv_w"].to(DEV), lw["A_log"].to(DEV), lw["dt_bias"].to(DEV), lw["norm_w"].to(DEV), 1e-6, DIMS)
    pool, states = pool_with_states(g_, 4)
    pool2 = wl.StateSlots(pool.S.shape[0], 2, H, DK, DV, C, K, device=DEV)
    pool2.S.copy_(pool.S)
    pool2.conv.copy_(pool.conv)
    states2 = pool2.views(range(2, 6))
    packed = backend.deltanet_prefill(*cols(y), states, 1, cu, *args)
    alone = torch.cat([backend.deltanet_prefill(*(t[lo:hi] for t in cols(y)), [st], 1, [0, hi - lo], *args)
                       for st, lo, hi in zip(states2, cu, cu[1:]) if hi > lo])
    assert torch.equal(packed, alone)
    assert torch.equal(pool.S, pool2.S) and torch.equal(pool.conv, pool2.conv)
