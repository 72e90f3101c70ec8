"""The allocation-free paged decode (rk_paged_decode_noalloc, called through the C ABI) against the workspace entry
point (rk_paged_decode) on the same inputs: bit-identical outputs (the same kernels and partition; only the address
of the partials differs), on two calls in a row, the second with a smaller batch, and with a gate read in place;
and captured in a HIP graph (after one eager call on the device, which resolves the scratch address and the
kernels' LDS limits), replayed three times with eager calls in between. Shapes whose partials exceed the fixed
scratch are refused before any launch."""
import pytest
import torch

import workloads as wl
from native import kernels

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def args_of(c, out, kernels_mod):
    B, Hq, d = c.q.shape
    NB, bs, Hkv, _ = c.k_pool.shape
    return (out.data_ptr(), c.q.data_ptr(), c.k_pool.data_ptr(), c.v_pool.data_ptr(),
            kernels_mod.DTYPE_CODES[c.k_pool.dtype], c.tables.data_ptr(), c.lens.data_ptr(), B, Hq, Hkv, d, bs,
            c.tables.shape[1], NB, int(c.window or 0), c.gate.data_ptr(), c.gate.stride(0))


def test_noalloc_equals_workspace_entry_point(backend):
    lib = backend.lib
    stream = torch.cuda.current_stream().cuda_stream
    assert lib.lib.rk_paged_decode_noalloc_max_bytes() == 16 << 20
    cases = [wl.c3_paged_decode(), wl.paged_decode_case([1, 7, 16, 33, 300], 32, 8, 2, 256, 16, torch.bfloat16,
                                                         seed=13)]
    for i, case in enumerate(cases):                  # batch 64, then batch 5 (the scratch keeps the last contents)
        c = case.to(DEV)
        B, Hq, d = c.q.shape
        want = torch.empty(B, Hq, d, device=DEV)
        got = torch.full((B, Hq, d), float("nan"), device=DEV)
        a = args_of(c, want, kernels)
        need = lib.lib.rk_paged_decode_workspace_bytes(B, Hq, a[9], d, a[11], a[12])
        ws = torch.empty(need, dtype=torch.uint8, device=DEV)
        lib.call("rk_paged_decode", *a, ws.data_ptr(), need, stream)
        lib.call("rk_paged_decode_noalloc", *args_of(c, got, kernels), stream)
        torch.cuda.synchronize()
        assert torch.equal(got, want), f"call {i}"
        assert torch.isfinite(got).all()


def test_noalloc_refuses_partials_beyond_its_scratch(backend):
    """Batch 1024 at 4 kv-heads x 256 needs 21 MB of partials: refused with RK_ERR_WORKSPACE, nothing launched."""
    lib = backend.lib
    B, Hq, Hkv, d = 1024, 16, 4, 256
    q = torch.zeros(B, Hq, d, device=DEV)
    pool = torch.zeros(4, 16, Hkv, d, dtype=torch.bfloat16, device=DEV)
    tables = torch.zeros(B, 1, dtype=torch.int32, device=DEV)
    lens = torch.ones(B, dtype=torch.int32, device=DEV)
    out = torch.zeros(B, Hq, d, device=DEV)
    need = lib.lib.rk_paged_decode_workspace_bytes(B, Hq, Hkv, d, 16, 1)
    assert need > lib.lib.rk_paged_decode_noalloc_max_bytes()
    rc = lib.lib.rk_paged_decode_noalloc(out.data_ptr(), q.data_ptr(), pool.data_ptr(), pool.data_ptr(), 1,
                                         tables.data_ptr(), lens.data_ptr(), B, Hq, Hkv, d, 16, 1, 4, 0, None, 0,
                                         torch.cuda.current_stream().cuda_stream)
    assert rc == 3 and b"scratch" in lib.lib.rk_last_error()
    torch.cuda.synchronize()
    assert torch.equal(out, torch.zeros_like(out))


def test_noalloc_captured_in_a_graph(backend):
    """The callers rk_paged_decode_noalloc is for include code under HIP graph capture: captured once (after an eager
    call on this device), every replay gives rk_paged_decode's bits, with eager calls of both entry points (which
    share the scratch and the workspace) between the replays."""
    lib = backend.lib
    c = wl.c3_paged_decode().to(DEV)
    B, Hq, d = c.q.shape
    want = torch.empty(B, Hq, d, device=DEV)
    a = args_of(c, want, kernels)
    need = lib.lib.rk_paged_decode_workspace_bytes(B, Hq, a[9], d, a[11], a[12])
    ws = torch.empty(need, dtype=torch.uint8, device=DEV)
    lib.call("rk_paged_decode", *a, ws.data_ptr(), need, torch.cuda.current_stream().cuda_stream)
    got = torch.full((B, Hq, d), float("nan"), device=DEV)
    lib.call("rk_paged_decode_noalloc", *args_of(c, got, kernels), torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert torch.equal(got, want)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        lib.call("rk_paged_decode_noalloc", *args_of(c, got, kernels), torch.cuda.current_stream().cuda_stream)
    other = wl.paged_decode_case([1, 7, 16, 33, 300], 32, 8, 2, 256, 16, torch.bfloat16, seed=13).to(DEV)
    o2 = torch.empty(other.q.shape, device=DEV)
    for rep in range(3):
        got.fill_(float("nan"))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(got, want), f"replay {rep}"
        lib.call("rk_paged_decode_noalloc", *args_of(other, o2, kernels), torch.cuda.current_stream().cuda_stream)
        lib.call("rk_paged_decode", *a, ws.data_ptr(), need, torch.cuda.current_stream().cuda_stream)
        torch.cuda.synchronize()
