"""HIP graph replays of the launches that keep state between calls (the linears' arrival counters, the paged decode's
workspace, the chunked delta rule's workspace): a chain of a residual linear with tile sums of squares, the RMSNorm
fused into the next linear, the SwiGLU down projection with its sums, the same MLP as rms_norm_swiglu then the plain
down projection (equal bits), a bf16 swiglu (K-split, counters), and config-3 paged decode with the gate,
captured once and replayed three times with eager calls of the same launches (which share the counters) in between;
and two chunked-delta calls on different inputs through one workspace, the second consuming the first's state.
Every replay must give the eager bits: the counters come back to zero after every launch, nothing in the chain is a
memset, and no launch starts before the one it depends on has finished."""
import pytest
import torch

import quant
import workloads as wl

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def test_decode_launch_chain_replays_bit_identical():
    from native import kernels
    g = torch.Generator().manual_seed(31)
    w_out = quant.quantize(torch.randn(2048, 2048, generator=g) * 0.02, "int4").to(DEV)
    w_gu = quant.quantize(torch.randn(12288, 2048, generator=g) * 0.02, "int4").to(DEV)
    w_dn = quant.quantize(torch.randn(2048, 6144, generator=g) * 0.02, "int4").to(DEV)
    o = torch.randn(8, 2048, generator=g).to(DEV)
    h0 = torch.randn(8, 2048, generator=g).to(DEV)
    nw = (1.0 + 0.1 * torch.randn(2048, generator=g)).to(DEV)
    c = wl.c3_paged_decode().to(DEV)

    w_gu_bf = (torch.randn(12288, 2048, generator=g) * 0.02).to(torch.bfloat16).to(DEV)   # K-split: counters

    def chain():
        h, ss = kernels.linear_ss(o, w_out, residual=h0)
        gu = kernels.rms_norm_linear(h, ss, nw, 1e-6, w_gu)
        h2, ss2 = kernels.silu_mul_linear_ss(gu[:, :6144], gu[:, 6144:], w_dn, residual=h)
        act = kernels.rms_norm_swiglu(h, ss, nw, 1e-6, w_gu)
        h3, ss3 = kernels.linear_ss(act, w_dn, residual=h)
        act_bf = kernels.swiglu(o, w_gu_bf)
        att = kernels.paged_decode(c.q, c.k_pool, c.v_pool, c.tables, c.lens, c.block_size, gate=c.gate)
        return h, ss, gu, h2, ss2, act, h3, ss3, act_bf, att

    want = [t.clone() for t in chain()]
    torch.cuda.synchronize()
    assert torch.equal(want[6], want[3]) and torch.equal(want[7], want[4])   # swiglu then down == the fused down
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        chain()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        outs = chain()
    for rep in range(3):
        graph.replay()
        torch.cuda.synchronize()
        for name, got, ref in zip(("h", "ss", "gate_up", "h2", "ss2", "swiglu", "h3", "ss3", "swiglu_bf16",
                                   "attention"), outs, want):
            assert torch.equal(got, ref), f"replay {rep}: {name}"
        eager = chain()                                  # the same launches between replays (shared counters)
        torch.cuda.synchronize()
        for got, ref in zip(eager, want):
            assert torch.equal(got, ref)


def test_replay_after_the_workspace_grew():
    """A graph captured while the shared workspace was small keeps writing to that buffer on every replay; when an
    eager call needs a larger one, the old buffer must stay allocated (never handed out again), and replays and
    eager calls must both keep giving the captured bits."""
    from native import kernels
    c = wl.c1_paged_decode().to(DEV)

    def decode():
        return kernels.paged_decode(c.q, c.k_pool, c.v_pool, c.tables, c.lens, c.block_size, gate=c.gate)

    want = decode().clone()
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        decode()
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = decode()
    old = kernels.workspace(c.q.device, 1)
    grown = kernels.workspace(c.q.device, old.numel() * 4)          # an eager call needing more: a new buffer
    assert grown.data_ptr() != old.data_ptr()
    junk = [torch.full((old.numel() // 4,), float("nan"), device=DEV) for _ in range(4)]   # allocations after it
    for rep in range(3):
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, want), f"replay {rep}"
        assert all(torch.isnan(j).all() for j in junk)              # the replay wrote nothing into them
        assert torch.equal(decode(), want)                          # eager, on the grown buffer


def test_chunked_delta_calls_replay_in_order():
    """Two config-4-sized rk_gated_delta_chunked calls on different inputs, both on one workspace (each call's prep
    writes the T / coefficient records its scan reads) and one state (the second call consumes what the first
    leaves), captured in one HIP graph twice over (A, B, A, B). Every replay gives the eager bits. A replay in which
    a call's prep started while the previous call's scan was still reading the workspace, or a scan before the
    previous scan had written the state, would change them: the inputs differ, so the records differ."""
    from native import kernels
    from native.rocm_native import load
    lib = load()
    g = torch.Generator().manual_seed(43)
    cases = [wl.c4_chunked_delta(seed=s).to(DEV) for s in (41, 42)]
    N, H, dk = cases[0].q.shape
    dv = cases[0].v.shape[2]
    cu = cases[0].cu_seqlens
    cuc = [0]
    for lo, hi in zip(cu, cu[1:]):
        cuc.append(cuc[-1] + -(-(hi - lo) // kernels.DELTA_CHUNK))
    n = len(cu) - 1
    meta = torch.tensor(cu + cuc, dtype=torch.int32).to(DEV)
    ws = torch.empty(lib.lib.rk_gated_delta_workspace_bytes(cuc[-1], H), dtype=torch.uint8, device=DEV)
    S0 = (0.05 * torch.randn(n, H, dk, dv, generator=g)).to(DEV)
    S = S0.clone()
    outs = [torch.empty(N, H, dv, device=DEV) for _ in range(4)]

    def call(c, out):
        lib.call("rk_gated_delta_chunked", out.data_ptr(), S.data_ptr(), S.stride(0), c.q.data_ptr(), c.k.data_ptr(),
                 c.v.data_ptr(), 1, c.beta.data_ptr(), c.g.data_ptr(), meta.data_ptr(), meta.data_ptr() + 4 * (n + 1),
                 None, n, cuc[-1], H, dk, dv, ws.data_ptr(), ws.numel(), torch.cuda.current_stream().cuda_stream)

    def chain():
        for i in range(4):
            call(cases[i % 2], outs[i])

    chain()
    torch.cuda.synchronize()
    want = [o.clone() for o in outs] + [S.clone()]
    assert not torch.equal(want[0], want[2])              # the second A call starts from another state
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        S.copy_(S0)
        chain()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        chain()
    for rep in range(3):
        S.copy_(S0)
        ws.fill_(0xFF)                                    # stale records: NaN patterns, never read
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for i, (got, ref) in enumerate(zip(outs + [S], want)):
            assert torch.equal(got, ref), f"replay {rep}: {'output ' + str(i) if i < 4 else 'state'}"
        S.copy_(S0)
        chain()                                           # the same launches eagerly between replays
        torch.cuda.synchronize()
        for got, ref in zip(outs + [S], want):
            assert torch.equal(got, ref)
