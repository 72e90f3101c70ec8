"""Parity of the rest of a decode step (rk_rms_norm, rk_layer_norm, rk_rope, rk_silu_mul; RocmBackend.rms_norm /
layer_norm / rope / silu_mul / swiglu / prepare) with the oracle's restatement of the reference's ops
(oracle/ops_ref.py: src/ops.py:7-54, 107-110), and a whole MLP block and attention-input block of a decode step
composed from backend calls against the same composition on the oracle.

Bar: fp32 outputs within 1e-5 relative (max |diff| / max |ref|). Edge cases: D from 1 to 12290 (one chunk per lane to
sixteen; D not a multiple of 256 or of 4; rows past 4096 values), bf16 inputs and weights read as stored, strided and
unaligned rows, large positions, F not a multiple of 4 (the scalar path), the two halves of one projection read in
place."""
import pytest
import torch

import quant
from helpers import rel_err
from oracle import ops_ref, quant_ref

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
TOL = 1e-5


@pytest.fixture(scope="module")
def backend():
    from backend.rocm import RocmBackend
    return RocmBackend(DEV)


@pytest.mark.parametrize("D", [4, 128, 256, 1000, 2048, 4096])
@pytest.mark.parametrize("kind", ["rms", "layer"])
def test_row_norms(backend, kind, D):
    g = torch.Generator().manual_seed(D)
    x = torch.randn(37, D, generator=g) * 2 + 0.5
    w = torch.randn(D, generator=g)
    ref = ops_ref.rms_norm if kind == "rms" else ops_ref.layer_norm
    fn = backend.rms_norm if kind == "rms" else backend.layer_norm
    assert rel_err(fn(x.to(DEV), w.to(DEV), 1e-6), ref(x, w, 1e-6)) < TOL
    # bf16 x and w read as stored; 3-D input; rows strided (every other row of a wider buffer)
    xb, wb = x.to(torch.bfloat16), w.to(torch.bfloat16)
    assert rel_err(fn(xb.to(DEV), wb.to(DEV), 1e-5), ref(xb, wb, 1e-5)) < TOL
    x3 = x.view(37, 1, D)
    assert fn(x3.to(DEV), w.to(DEV), 1e-6).shape == (37, 1, D)
    wide = torch.randn(37, 2 * D + 8, generator=g)
    view = wide.to(DEV)[:, 4:4 + D]
    assert rel_err(fn(view, w.to(DEV), 1e-6), ref(wide[:, 4:4 + D], w, 1e-6)) < TOL


@pytest.mark.parametrize("D", [1, 5, 4097, 4100, 8192, 12290])
@pytest.mark.parametrize("kind", ["rms", "layer"])
def test_row_norms_of_any_length(backend, kind, D):
    """Rows the register kernel does not take (longer than 4096, a length not a multiple of 4, unaligned): the
    reference's ops have no limit on D (src/ops.py:7-24)."""
    g = torch.Generator().manual_seed(100 + D)
    x = torch.randn(9, D, generator=g) * 3 - 0.25
    w = torch.randn(D, generator=g)
    ref = ops_ref.rms_norm if kind == "rms" else ops_ref.layer_norm
    fn = backend.rms_norm if kind == "rms" else backend.layer_norm
    assert rel_err(fn(x.to(DEV), w.to(DEV), 1e-6), ref(x, w, 1e-6)) < TOL
    xb, wb = x.to(torch.bfloat16), w.to(torch.bfloat16)
    assert rel_err(fn(xb.to(DEV), wb.to(DEV), 1e-5), ref(xb, wb, 1e-5)) < TOL
    wide = torch.randn(9, 2 * D + 3, generator=g)   # rows strided by an odd number of elements, start unaligned
    view = wide.to(DEV)[:, 1:1 + D]
    assert rel_err(fn(view, w.to(DEV), 1e-6), ref(wide[:, 1:1 + D], w, 1e-6)) < TOL


def test_row_norm_of_constant_rows(backend):
    """LayerNorm of a constant row is 0 (the centering is exact); RMSNorm of a constant c is c / sqrt(c^2 + eps)."""
    x = torch.full((3, 512), 2.5)
    w = torch.ones(512)
    assert backend.layer_norm(x.to(DEV), w.to(DEV), 1e-5).abs().max().item() == 0.0
    assert rel_err(backend.rms_norm(x.to(DEV), w.to(DEV), 1e-6), ops_ref.rms_norm(x, w, 1e-6)) < 1e-7


@pytest.mark.parametrize("d,theta", [(64, 1e4), (128, 1e6), (256, 1e7)])
def test_rope(backend, d, theta):
    g = torch.Generator().manual_seed(d)
    T, H = 11, 6
    x = torch.randn(T, H, d, generator=g)
    pos = torch.tensor([0, 1, 2, 3, 100, 4095, 4096, 16383, 20000, 123457, 262143], dtype=torch.int32)
    got = backend.rope(x.to(DEV), pos.to(DEV), theta)
    assert rel_err(got, ops_ref.rope(x, pos, theta)) < TOL
    assert torch.equal(got[0].cpu(), x[0])                       # position 0 is the identity


@pytest.mark.parametrize("rows,F", [(1, 6144), (8, 6144), (3, 1001), (70, 512)])
def test_silu_mul(backend, rows, F):
    g_ = torch.Generator().manual_seed(F)
    g, u = torch.randn(rows, F, generator=g_) * 4, torch.randn(rows, F, generator=g_)
    assert rel_err(backend.silu_mul(g.to(DEV), u.to(DEV)), ops_ref.silu_mul(g, u)) < TOL
    y = torch.cat([g, u], dim=1).to(DEV)                         # the two halves of one projection, in place
    assert rel_err(backend.silu_mul(y[:, :F], y[:, F:]), ops_ref.silu_mul(g, u)) < TOL


@pytest.mark.parametrize("scheme", [None, "int8", "int4"])
def test_swiglu_and_prepare(scheme, backend):
    """prepare() applies the reference's policy; swiglu over the prepared [gate; up] weight equals the oracle's
    silu_mul of the dequantized weight's two halves."""
    from backend.rocm import RocmBackend
    be = RocmBackend(DEV, scheme=scheme)
    g_ = torch.Generator().manual_seed(7)
    F, K = 1536, 1024
    w = torch.randn(2 * F, K, generator=g_) * 0.05
    pw = be.prepare(w, "model.language_model.layers.0.mlp.gate_up.weight")
    emb = be.prepare(torch.randn(4096, K, generator=g_) * 0.05, "model.embed_tokens.weight")
    if scheme is None:
        assert pw.dtype == torch.bfloat16 and emb.dtype == torch.bfloat16
        deq = pw.float().cpu()
    else:
        assert isinstance(pw, quant.QuantTensor) and pw.scheme == scheme
        assert emb.scheme == "int8"                              # the tied embedding stays INT8 in both modes
        deq = quant_ref.dequantize(pw.scheme, pw.data.cpu(), pw.scales.cpu(),
                                   pw.mins.cpu() if pw.mins is not None else None)
    for M in (1, 8, 40):
        x = torch.randn(M, K, generator=g_)
        y = x @ deq.T
        assert rel_err(be.swiglu(x.to(DEV), pw), ops_ref.silu_mul(y[:, :F], y[:, F:])) < TOL


def test_mlp_block_of_a_decode_step(backend):
    """One decode step's MLP block at batch 8, Qwen3.5-2B widths, INT4: h + down(swiglu(rms_norm(h))) through the
    backend against the same composition on the oracle (the reference's decoder layer, src/models/qwen3_5.py)."""
    from backend.rocm import RocmBackend
    be = RocmBackend(DEV, scheme="int4")
    g_ = torch.Generator().manual_seed(11)
    H, I = 2048, 6144
    norm_w = 1.0 + 0.1 * torch.randn(H, generator=g_)
    gate_up = be.prepare(torch.randn(2 * I, H, generator=g_) * 0.02, "layers.0.mlp.gate_up.weight")
    down = be.prepare(torch.randn(H, I, generator=g_) * 0.02, "layers.0.mlp.down_proj.weight")
    deq = lambda q: quant_ref.dequantize(q.scheme, q.data.cpu(), q.scales.cpu(), q.mins.cpu())
    h = torch.randn(8, H, generator=g_)
    hd = h.to(DEV)
    got = be.linear(be.swiglu(be.rms_norm(hd, norm_w.to(DEV), 1e-6), gate_up), down, residual=hd)
    x = ops_ref.rms_norm(h, norm_w, 1e-6)
    y = x @ deq(gate_up).T
    want = quant_ref.linear(ops_ref.silu_mul(y[:, :I], y[:, I:]), deq(down), None, h)
    assert rel_err(got, want) < TOL
