"""A whole hybrid decode step through RocmBackend -- the sequence of backend calls of Qwen3_5Model.decode_batch
(src/models/qwen3_5.py:228-290): embedding, per layer RMSNorm, the attention layer (qkvg projection, fused q / k norm
+ partial RoPE + KV write, paged attention with the fused gate, o_proj + residual) or the DeltaNet layer (in_proj,
batched recurrent step on the pool's states, out_proj + residual), RMSNorm and the SwiGLU MLP, then the final norm
and the tied head -- against the same composition on the oracle (oracle/decode_ref.py), on a small 4-layer stack
(3 DeltaNet + 1 attention layer) with bf16 and INT4 (INT8 embedding) weights.

Bars: logits within 1e-5 relative (max |diff| / max |ref|); the DeltaNet states and conv tails the step writes
within 1e-5; the KV rows written equal the oracle's after rounding to bf16 except where the fp32 values straddle a
rounding boundary (at most one bf16 ulp)."""
import pytest
import torch

import quant
import workloads as wl
from helpers import rel_err
from oracle import decode_ref, quant_ref

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
TOL = 1e-5
SMALL = wl.HybridConfig(layers=4, hidden=256, intermediate=512, vocab=1000, Hq=8, Hkv=2, d=128, rot=32, theta=1e6,
                        H=4, dk=128, dv=128)


def device_weights(be, host: dict):
    """2-D weights through prepare() (the model's _w / _fused), vectors and conv taps fp32 (its _vec); and the fp32
    values the backend then holds, for the oracle."""
    dev, ref = {}, {}
    for name, w in host.items():
        if w.dim() == 2 and not name.endswith("conv1d.weight"):
            p = be.prepare(w, name)
            dev[name] = p
            if isinstance(p, quant.QuantTensor):
                ref[name] = quant_ref.dequantize(p.scheme, p.data.cpu(), p.scales.cpu(),
                                                 p.mins.cpu() if p.mins is not None else None)
            else:
                ref[name] = p.float().cpu()
        else:
            dev[name] = w.to(DEV)
            ref[name] = w
    return dev, ref


@pytest.mark.parametrize("scheme", [None, "int4"])
def test_hybrid_decode_step_matches_oracle(scheme):
    from backend.rocm import RocmBackend
    be = RocmBackend(DEV, scheme=scheme)
    cfg = SMALL
    wd, wh = device_weights(be, wl.hybrid_weights(cfg, seed=21))
    if scheme == "int4":
        assert wd["embed_tokens.weight"].scheme == "int8" and wd["layers.0.mlp.gate_up.weight"].scheme == "int4"
    lens = [5, 40, 17, 100]
    st = wl.HybridDecodeState(cfg, lens, DEV, seed=22)
    kh, vh = st.k.cpu(), st.v.cpu()
    Sh, convh = st.pool.S.cpu(), st.pool.conv.cpu()
    seq_index = torch.tensor([s.seq for s in st.seqs])
    layout = st.layout()
    slots, tables, lens_t, positions = (t.cpu() for t in layout)
    tokens = torch.tensor([3, 999, 0, 512])
    got = wl.hybrid_decode_step(be, wd, st, tokens.to(DEV), layout)
    want = decode_ref.hybrid_decode_step(cfg, wh, kh, vh, Sh, convh, seq_index, st.slot, slots, tables, lens_t,
                                         positions, tokens)
    assert got.shape == (4, cfg.vocab)
    assert rel_err(got, want) < TOL
    assert rel_err(st.pool.S, Sh) < TOL and rel_err(st.pool.conv, convh) < TOL
    rows = slots.long()
    for L in range(st.k.shape[0]):
        for pool, ref in ((st.k, kh), (st.v, vh)):
            g = pool[L].view(-1, cfg.Hkv, cfg.d)[rows.to(DEV)].float().cpu()
            r = ref[L].view(-1, cfg.Hkv, cfg.d)[rows].float()
            ulp = r.abs().clamp_min(1e-30) * 2.0 ** -7
            assert ((g - r).abs() <= ulp).all()
