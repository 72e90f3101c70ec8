"""HIP graph replays of the decode-step launches that keep state between calls (the linears' arrival counters, the
paged decode's workspace): a chain of a residual linear with tile sums of squares, the RMSNorm fused into the next
linear, the SwiGLU down projection with its sums, and config-3 paged decode with the gate, captured once and
replayed three times with eager calls of the same launches (which share the counters) in between. Every replay must
give the eager bits: the counters come back to zero after every launch, and nothing in the chain is a memset."""
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

    def chain():
        h, ss = kernels.linear_ss(o, w_out, residual=h0)
        gu = kernels.rms_norm_linear(h, ss, nw, 1e-6, w_gu)
        h2, ss2 = kernels.silu_mul_linear_ss(gu[:, :6144], gu[:, 6144:], w_dn, residual=h)
        att = kernels.paged_decode(c.q, c.k_pool, c.v_pool, c.tables, c.lens, c.block_size, gate=c.gate)
        return h, ss, gu, h2, ss2, att

    want = [t.clone() for t in chain()]
    torch.cuda.synchronize()
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
        for name, got, ref in zip(("h", "ss", "gate_up", "h2", "ss2", "attention"), outs, want):
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
