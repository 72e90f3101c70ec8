"""The block-quantized weight format (metal-inference-engine_amd/quant.py, a restatement of src/quant.py) and the
oracle's dequantize (oracle/quant_ref.py), on the CPU: the reference's own known answers (tests/test_quant.py:25-44
of the reference: the INT4 packing byte, the half-step error bound, row stacking) plus float64 arithmetic."""
import numpy as np
import pytest
import torch

import quant
from oracle import quant_ref


def deq(q: quant.QuantTensor) -> torch.Tensor:
    return quant_ref.dequantize(q.scheme, q.data, q.scales, q.mins, q.block)


def test_int4_packing_order():
    """[1, -1] * 16: min -1, max 1, scale 2/15 -> q = 15 for +1 (low nibble of byte 0), 0 for -1 (high nibble)."""
    q = quant.quantize(torch.tensor([[1.0, -1.0] * 16]), "int4")
    assert q.data[0, 0].item() == 0x0F
    assert (deq(q) - torch.tensor([[1.0, -1.0] * 16])).abs().max() < 1e-3     # fp16 scale: 15 * fp16(2/15) - 1


@pytest.mark.parametrize("scheme", ["int8", "int4"])
def test_dequant_error_within_half_a_step(scheme):
    torch.manual_seed(0)
    w = torch.randn(64, 256) * 0.05 + 0.02
    q = quant.quantize(w, scheme)
    err = (deq(q) - w).abs().view(64, -1, 32)
    step = q.scales.float()[..., None]
    assert (err <= step / 2 * 1.01 + 1e-6).all()
    assert q.nbytes < w.numel() * 2


def test_dequantize_is_the_block_formula_in_float64():
    """The oracle's dequantize against the definition computed independently in float64 (element 2j low nibble)."""
    g = torch.Generator().manual_seed(1)
    w = torch.randn(8, 96, generator=g)
    for scheme in ("int8", "int4"):
        q = quant.quantize(w, scheme)
        s = q.scales.double().repeat_interleave(32, dim=1)
        if scheme == "int8":
            want = q.data.double() * s
        else:
            d = q.data.numpy().astype(np.int64)
            codes = np.empty((8, 96), dtype=np.int64)
            codes[:, 0::2], codes[:, 1::2] = d & 15, d >> 4
            want = torch.tensor(codes, dtype=torch.float64) * s + q.mins.double().repeat_interleave(32, dim=1)
        assert torch.allclose(deq(q).double(), want, rtol=1e-7, atol=1e-9)


def test_stacking_rows_equals_quantizing_the_stack():
    g = torch.Generator().manual_seed(2)
    a, b = torch.randn(96, 128, generator=g), torch.randn(32, 128, generator=g)
    qa, qb, qab = quant.quantize(a, "int4"), quant.quantize(b, "int4"), quant.quantize(torch.cat([a, b]), "int4")
    st = quant.concat_rows([qa, qb])
    assert torch.equal(st.data, qab.data) and torch.equal(st.scales, qab.scales) and torch.equal(st.mins, qab.mins)
    sel = quant.select_rows(qab, torch.tensor([3, 100]))
    assert torch.equal(sel.data, qab.data[[3, 100]]) and sel.shape == (2, 128)


def test_quantize_in_row_chunks_is_bit_identical(monkeypatch):
    g = torch.Generator().manual_seed(3)
    w = torch.randn(40, 64, generator=g)
    for scheme in ("int8", "int4"):
        whole = quant.quantize(w, scheme)
        monkeypatch.setattr(quant, "CHUNK", 100)
        parts = quant.quantize(w, scheme)
        monkeypatch.setattr(quant, "CHUNK", 1 << 24)
        assert torch.equal(parts.data, whole.data) and torch.equal(parts.scales, whole.scales)


def test_policy_groups_and_int8_exceptions():
    """The reference's own expectations for the INT4 precision policy (tests/test_quant.py:58-73 of the reference):
    checkpoint component names and fused names map to one group; a kept fused tensor keeps all its components INT8;
    the tied embedding stays INT8."""
    ck = "model.language_model."
    assert (quant.policy_group(ck + "layers.3.self_attn.q_proj.weight")
            == quant.policy_group(ck + "layers.3.self_attn.k_proj.weight")
            == quant.policy_group("layers.3.self_attn.qkvg.weight") == "layers.3.attn_in")
    assert (quant.policy_group(ck + "layers.5.linear_attn.in_proj_z.weight")
            == quant.policy_group("layers.5.linear_attn.in_proj.weight") == "layers.5.linear_in")
    assert (quant.policy_group(ck + "layers.3.mlp.gate_proj.weight")
            == quant.policy_group("layers.3.mlp.gate_up.weight") == "layers.3.mlp_in")
    assert quant.policy_group(ck + "layers.3.mlp.down_proj.weight") == "layers.3.mlp.down_proj.weight"
    assert (quant.policy_group("model.layers.3.self_attn.k_proj.weight")
            == quant.policy_group("layers.3.self_attn.qkv.weight") == "layers.3.attn_in")
    keep = frozenset({"layers.3.self_attn.qkvg.weight", "layers.0.linear_attn.in_proj.weight"})
    kept = ({quant.scheme_for(f"{ck}layers.3.self_attn.{c}_proj.weight", "int4", keep) for c in "qkv"}
            | {quant.scheme_for(f"{ck}layers.0.linear_attn.in_proj_{c}.weight", "int4", keep)
               for c in ("qkv", "z", "b", "a")})
    assert kept == {"int8"}
    assert quant.scheme_for(ck + "layers.3.mlp.down_proj.weight", "int4", keep) == "int4"
    assert quant.scheme_for("model.embed_tokens.weight", "int4") == "int8"
    assert quant.scheme_for("model.embed_tokens.weight", "int8") == "int8"
    assert quant.scheme_for(None, "int4") == "int4"


def test_load_policy(tmp_path):
    p = tmp_path / "policy.json"
    p.write_text('{"keep_int8": ["model.language_model.layers.2.mlp.up_proj.weight"]}')
    assert quant.load_policy(str(p)) == frozenset({"layers.2.mlp_in"})
    assert quant.load_policy(None) == frozenset()
