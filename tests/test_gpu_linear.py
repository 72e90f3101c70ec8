"""Parity of the decode-time linears (rk_linear_rows, rk_dequant_rows; RocmBackend.linear / embedding) with the
oracle's restatement of the reference's math (oracle/quant_ref.py: QuantTensor.dequantize, src/quant.py:45-56, then
y = x @ w.T + bias + residual in fp32, src/backend/metal.py:59-133).

Bars: dequantized rows bit-exact (q * scale, + min, each rounded, as the reference); linear outputs (fp32) within
1e-5 relative. Shapes: Qwen3.5-0.8B's qkvg / down / gate_up (the reference's own kernel test shapes,
tests/test_quant.py:46-55 there), Qwen3.5-2B's, and ragged ones (rows not a multiple of 64, K not a multiple of the
K-tile)."""
import pytest
import torch

import quant
from helpers import rel_err
from oracle import quant_ref

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
TOL = 1e-5


def weight(kind, N, K, seed):
    g = torch.Generator().manual_seed(seed)
    w = torch.randn(N, K, generator=g) * 0.05 + 0.01
    if kind == "bf16":
        return w.to(torch.bfloat16), w.to(torch.bfloat16).float()
    q = quant.quantize(w, kind)
    return q, quant_ref.dequantize(q.scheme, q.data, q.scales, q.mins)


def to_dev(w):
    return w.to(DEV) if isinstance(w, quant.QuantTensor) else w.to(DEV)


@pytest.mark.parametrize("kind", ["bf16", "int8", "int4"])
def test_dequant_rows_bit_exact(backend, kind):
    from native import kernels
    w, deq = weight(kind, 300, 224, 1)
    wd = to_dev(w)
    assert torch.equal(kernels.dequantize(wd).cpu(), deq)
    rows = torch.tensor([299, 0, 17, 17, 150])
    assert torch.equal(kernels.dequantize(wd, rows=rows.to(DEV)).cpu(), deq[rows])
    assert torch.equal(backend.embedding(wd, rows.to(DEV)).cpu(), deq[rows])


# 33000 x 1024 takes four 16-row tiles per workgroup (ragged last group), (100, 96) and (65, 2080) the unaligned
# parameter loads and a last K-split of one block; (70001, 2048) is a long matrix (INT8 at up to 8 rows: the
# persistent kernel, a ragged last tile)
SHAPES = [(5120, 1024), (1024, 3584), (7168, 1024), (8224, 2048), (2048, 6144), (33000, 1024), (100, 96), (65, 2080),
          (70001, 2048)]


@pytest.mark.parametrize("N,K", SHAPES)
@pytest.mark.parametrize("kind", ["bf16", "int8", "int4"])
def test_linear_rows_matches_dequantized_reference(backend, kind, N, K):
    w, deq = weight(kind, N, K, N + K)
    g = torch.Generator().manual_seed(K)
    wd = to_dev(w)
    worst = 0.0
    for M, with_b, with_r in ((1, False, True), (3, True, False), (8, True, True), (16, False, False),
                              (20, True, True), (32, False, True)):
        x = torch.randn(M, K, generator=g)
        b = torch.randn(N, generator=g) if with_b else None
        r = torch.randn(M, N, generator=g) if with_r else None
        want = quant_ref.linear(x, deq, b, r)
        got = backend.linear(x.to(DEV), wd, None if b is None else b.to(DEV), None if r is None else r.to(DEV))
        e = rel_err(got, want)
        worst = max(worst, e)
        assert e < TOL, f"M {M}: rel {e:.2e}"
    print(f"linear {kind} {N}x{K}: worst rel {worst:.2e}")


@pytest.mark.parametrize("kind", ["bf16", "int8", "int4"])
def test_prefill_sized_linear_goes_through_dequantized_gemm(backend, kind):
    w, deq = weight(kind, 1000, 512, 9)
    g = torch.Generator().manual_seed(9)
    x, r = torch.randn(70, 512, generator=g), torch.randn(70, 1000, generator=g)
    got = backend.linear(x.to(DEV), to_dev(w), residual=r.to(DEV))
    assert rel_err(got, quant_ref.linear(x, deq, None, r)) < TOL


def test_rows_are_independent_of_the_batch(backend):
    """A row's output does not depend on the other rows launched with it: the reference's exact targets hold batched
    runs equal to sequential ones (tests/serving_targets.py:42)."""
    w, _ = weight("int4", 2048, 2048, 4)
    wd = to_dev(w)
    x = torch.randn(16, 2048, generator=torch.Generator().manual_seed(4)).to(DEV)
    full = backend.linear(x, wd)
    for i in (0, 7, 15):
        assert torch.equal(backend.linear(x[i:i + 1], wd), full[i:i + 1])


@pytest.mark.parametrize("N,K", [(2048, 6144), (1024, 3584), (640, 2048), (96, 256)])
@pytest.mark.parametrize("kind", ["bf16", "int8", "int4"])
def test_silu_mul_fused_into_the_linear(backend, kind, N, K):
    """silu_mul_linear (rk_linear_rows_ex, RK_X_SILU_MUL) over the two halves of one [M, 2K] gate_up output read in
    place == linear(silu_mul(gate, up)) on the oracle; more than 8 rows take the two-launch path (same bar); a fused
    row does not depend on the batch."""
    from oracle import ops_ref
    w, deq = weight(kind, N, K, 7 * N + K)
    g = torch.Generator().manual_seed(K)
    wd = to_dev(w)
    for M in (1, 5, 8, 12):
        y = torch.randn(M, 2 * K, generator=g) * 2
        r = torch.randn(M, N, generator=g)
        want = quant_ref.linear(ops_ref.silu_mul(y[:, :K], y[:, K:]), deq, None, r)
        yd = y.to(DEV)
        got = backend.silu_mul_linear(yd[:, :K], yd[:, K:], wd, residual=r.to(DEV))
        assert rel_err(got, want) < TOL, f"M {M}"
    yd = yd[:8]
    full = backend.silu_mul_linear(yd[:, :K], yd[:, K:], wd)
    assert torch.equal(backend.silu_mul_linear(yd[3:4, :K], yd[3:4, K:], wd), full[3:4])


@pytest.mark.parametrize("F,K", [(6144, 2048), (3584, 1024), (1024, 3072), (520, 2080), (48, 256)])
@pytest.mark.parametrize("kind", ["bf16", "int8", "int4"])
def test_swiglu_rows(backend, kind, F, K):
    """rk_swiglu_rows (RocmBackend.swiglu): silu(x gate^T) * (x up^T) over the stacked [gate; up] weight in one
    launch == the oracle's linear then silu_mul within 1e-5 at 1, 5, 8, 16 and 20 rows (20: two launches; 33: the
    GEMM then silu_mul); a row's result does not depend on the batch; where the fused silu * up down projection
    covers the shape (M <= 8, F % 256 == 0), swiglu then the down projection equals the plain linear then that fused
    projection bit for bit (the gate / up sums are the linear's, and silu * up is computed in the same form)."""
    from native import kernels
    from oracle import ops_ref
    w, deq = weight(kind, 2 * F, K, 3 * F + K)
    wdn, _ = weight("int4", 256, F, F) if F % 32 == 0 else weight("bf16", 256, F, F)
    wd, wdnd = to_dev(w), to_dev(wdn)
    g = torch.Generator().manual_seed(F + K)
    x33 = torch.randn(33, K, generator=g)
    got_by_m = {}
    for M in (8, 1, 5, 16, 20, 33):
        x = x33[:M]
        y = quant_ref.linear(x, deq, None, None)
        want = ops_ref.silu_mul(y[:, :F], y[:, F:])
        got = backend.swiglu(x.to(DEV), wd)
        assert got.shape == (M, F)
        assert rel_err(got, want) < TOL, f"M {M}"
        got_by_m[M] = got.cpu()
        if M <= 8 and F % 256 == 0:
            xd = x.to(DEV)
            gu = kernels.linear(xd, wd)
            two = kernels.silu_mul_linear(gu[:, :F], gu[:, F:], wdnd)
            assert torch.equal(kernels.linear(got, wdnd), two), f"M {M}"
    assert torch.equal(got_by_m[1][0], got_by_m[8][0])
    assert torch.equal(got_by_m[5], got_by_m[8][:5])


@pytest.mark.parametrize("kind", ["int4", "int8", "bf16"])
def test_rms_norm_swiglu_is_the_decode_mlp(backend, kind):
    """The decode step's MLP at Qwen3.5-2B widths: rms_norm_swiglu (the norm from the producer's tile sums while x is
    staged, silu * up in the epilogue) then the down projection with its tile sums == rms_norm_linear over gate_up
    then silu_mul_linear_ss bit for bit (both outputs and sums) at 1, 5 and 8 rows, and the oracle's
    h + down(silu_mul(linear(rms_norm(h)))) within 1e-5; beyond 8 rows the separate norm runs (same bar)."""
    from native import kernels
    from oracle import ops_ref
    F, K = 6144, 2048
    w, deq = weight(kind, 2 * F, K, 11)
    wdn, deq_dn = weight(kind, K, F, 12)
    wp, _ = weight("int4", K, 2048, 13)                 # the producer of h
    wd, wdnd, wpd = to_dev(w), to_dev(wdn), to_dev(wp)
    g = torch.Generator().manual_seed(14)
    nw = (1.0 + 0.1 * torch.randn(K, generator=g)).to(DEV)
    o12, r12 = torch.randn(12, 2048, generator=g), torch.randn(12, K, generator=g)
    for M in (8, 1, 5, 12):
        h, ss = kernels.linear_ss(o12[:M].to(DEV), wpd, residual=r12[:M].to(DEV))
        act = kernels.rms_norm_swiglu(h, ss, nw, 1e-6, wd)
        y, ss2 = kernels.linear_ss(act, wdnd, residual=h)
        want_act = ops_ref.silu_mul(*quant_ref.linear(ops_ref.rms_norm(h.cpu(), nw.cpu(), 1e-6), deq, None,
                                                      None).split(F, dim=1))
        assert rel_err(act, want_act) < TOL, f"M {M}"
        assert rel_err(y, quant_ref.linear(want_act, deq_dn, None, h.cpu())) < TOL, f"M {M}"
        if M <= 8:
            gu = kernels.rms_norm_linear(h, ss, nw, 1e-6, wd)
            y2, ss3 = kernels.silu_mul_linear_ss(gu[:, :F], gu[:, F:], wdnd, residual=h)
            assert torch.equal(y, y2) and torch.equal(ss2, ss3), f"M {M}"


def tile_sums(y):
    """Sums of squares of y's 16-column tiles [M, ceil(N / 16)] (the last tile zero-padded)."""
    M, N = y.shape
    pad = torch.zeros(M, -(-N // 16) * 16)
    pad[:, :N] = y
    return (pad * pad).view(M, -1, 16).sum(-1)


@pytest.mark.parametrize("N,K", [(2048, 2048), (2048, 6144), (2064, 1024), (100, 96), (8224, 2048), (65552, 1024)])
@pytest.mark.parametrize("kind", ["bf16", "int8", "int4"])
def test_linear_with_tile_sums_of_squares(backend, kind, N, K):
    """rk_linear_rows_ex2 with ss_out: y bit-identical to the plain launch, and the tile sums of squares within 1e-6
    of the fp64 sums of the same y (S == 1 and S > 1 epilogues; N not a multiple of 16 or 32)."""
    from native import kernels
    w, _ = weight(kind, N, K, 3 * N + K)
    wd = to_dev(w)
    g = torch.Generator().manual_seed(N)
    for M in (1, 5, 8, 16):
        x, r = torch.randn(M, K, generator=g), torch.randn(M, N, generator=g)
        y, ss = kernels.linear_ss(x.to(DEV), wd, residual=r.to(DEV))
        assert torch.equal(y.cpu(), kernels.linear_rows(x.to(DEV), wd, residual=r.to(DEV)).cpu())
        assert ss.shape == (M, -(-N // 16))
        assert rel_err(ss, tile_sums(y.cpu().double()).float()) < 1e-6


@pytest.mark.parametrize("kind", ["bf16", "int8", "int4"])
@pytest.mark.parametrize("N,K", [(8224, 2048), (12288, 2048), (6144, 1024), (16384, 256), (248320, 2048)])
def test_rms_norm_fused_into_the_linear(backend, kind, N, K):
    """RK_X_RMS_NORM: linear(rms_norm(h)) in one launch from the tile sums of squares of the linear that wrote h,
    against the oracle's rms_norm then linear (1e-5), for 1, 5 and 8 rows; a row's result does not depend on the
    batch (bit-identical at M = 1 and M = 8); beyond 8 rows (and for N > 16384, the head) the two-launch form
    runs."""
    from native import kernels
    from oracle import ops_ref
    w, deq = weight(kind, N, K, N + 7 * K)
    wp, _ = weight("int4", K, 2048, K)                  # the producer of h
    wd, wpd = to_dev(w), to_dev(wp)
    g = torch.Generator().manual_seed(K + 1)
    nw = (1.0 + 0.1 * torch.randn(K, generator=g)).to(DEV)
    o8, r8 = torch.randn(8, 2048, generator=g), torch.randn(8, K, generator=g)
    got_by_m = {}
    for M in (8, 1, 5, 12):                             # 12: the two-launch form
        o, r = o8[:M] if M <= 8 else torch.randn(M, 2048, generator=g), r8[:M] if M <= 8 else torch.randn(M, K, generator=g)
        h, ss = kernels.linear_ss(o.to(DEV), wpd, residual=r.to(DEV))
        got = kernels.rms_norm_linear(h, ss, nw, 1e-6, wd)
        want = quant_ref.linear(ops_ref.rms_norm(h.cpu(), nw.cpu(), 1e-6), deq, None, None)
        assert rel_err(got, want) < TOL
        got_by_m[M] = got.cpu()
    assert torch.equal(got_by_m[1][0], got_by_m[8][0])


@pytest.mark.parametrize("N,K", [(248320, 2048), (65541, 1024), (131072, 2048)])
def test_long_int8_matrix_on_the_persistent_grid(backend, N, K):
    """INT8 matrices of 65536+ rows at up to 8 activation rows (the tied LM head, N = 248320) run on one persistent
    workgroup per CU streaming whole 16-row tiles: against the dequantized reference within 1e-5 with bias and
    residual, the tile sums of squares within 1e-6 of the fp64 sums of y, a row's result independent of the batch
    (M = 1 and M = 8 bit-identical), and a ragged last tile."""
    from native import kernels
    w, deq = weight("int8", N, K, N + 3 * K)
    wd = to_dev(w)
    g = torch.Generator().manual_seed(N % 1000)
    x8 = torch.randn(8, K, generator=g)
    b, r8 = torch.randn(N, generator=g), torch.randn(8, N, generator=g)
    rows = {}
    for M in (8, 3, 1):
        x, r = x8[:M], r8[:M]
        want = quant_ref.linear(x, deq, b, r)
        got = backend.linear(x.to(DEV), wd, b.to(DEV), r.to(DEV))
        e = rel_err(got, want)
        print(f"long int8 {N}x{K}, M {M}: rel {e:.2e}")
        assert e < TOL
        y, ss = kernels.linear_ss(x.to(DEV), wd, residual=r.to(DEV))
        assert rel_err(ss, tile_sums(y.cpu().double()).float()) < 1e-6
        rows[M] = got.cpu()
    assert torch.equal(rows[1][0], rows[8][0]) and torch.equal(rows[3], rows[8][:3])
