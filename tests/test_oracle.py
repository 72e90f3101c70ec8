"""Pins of the CPU oracle (oracle/) — against float64 brute force, the committed golden fixtures (tests/golden/,
written by make_golden.py from float64 definitions and from transformers' Qwen3.5 routines), library routines, and
the invariants the reference's own tests hold. Each check is chosen so that a plausible slip (mask offset, GQA head
mapping, missing decay, transposed operand, wrong substitution order) fails it."""
import os
from pathlib import Path

import numpy as np
import pytest
import torch

from helpers import SlotState, rel_err
from oracle import backend_ref, brute, ops_ref

GOLD = Path(__file__).resolve().parent / "golden"
os.environ.setdefault("HF_HUB_OFFLINE", "1")


def t(a, dtype=torch.float32):
    return torch.tensor(np.asarray(a), dtype=dtype)


# ---------------------------------------------------------------- attention (ops.attention, src/ops.py:65-104)

@pytest.mark.parametrize("T,S,Hq,Hkv,d,window", [(1, 1, 8, 2, 32, None), (1, 300, 8, 2, 64, None),
                                                  (5, 5, 4, 2, 16, None), (6, 15, 4, 2, 16, None),
                                                  (7, 40, 14, 2, 16, 9), (1, 50, 16, 4, 32, 16),
                                                  (3, 3, 4, 1, 8, 1)])
def test_attention_matches_float64_brute_force(T, S, Hq, Hkv, d, window):
    g = torch.Generator().manual_seed(T * 1000 + S)
    q, k, v = torch.randn(T, Hq, d, generator=g), torch.randn(S, Hkv, d, generator=g), torch.randn(S, Hkv, d, generator=g)
    got = ops_ref.attention(q, k, v, causal=True, window=window)
    want = brute.attention(q.numpy(), k.numpy(), v.numpy(), True, window)
    assert rel_err(got, want) < 2e-6


def test_attention_fixture():
    f = np.load(GOLD / "prefill_attention.npz")
    assert rel_err(ops_ref.attention(t(f["q"]), t(f["k"]), t(f["v"])), f["out_full"]) < 2e-6
    assert rel_err(ops_ref.attention(t(f["q"]), t(f["k"]), t(f["v"]), window=4), f["out_w4"]) < 2e-6


def test_one_key_returns_its_value():
    q, k, v = torch.randn(1, 8, 16), torch.randn(1, 2, 16), torch.randn(1, 2, 16)
    assert torch.equal(ops_ref.attention(q, k, v), v.repeat_interleave(4, dim=1))


def test_large_scores_stay_finite():
    g = torch.Generator().manual_seed(3)
    q = torch.randn(1, 8, 64, generator=g) * 30
    k, v = torch.randn(300, 2, 64, generator=g), torch.randn(300, 2, 64, generator=g)
    got = ops_ref.attention(q, k, v)
    assert torch.isfinite(got).all()
    assert rel_err(got, brute.attention(q.numpy(), k.numpy(), v.numpy())) < 1e-5


# ---------------------------------------------------------------- paged decode (torch_ref.py:75-88)

def test_paged_decode_fixture():
    f = np.load(GOLD / "paged_decode.npz")
    args = (t(f["q"]), t(f["k_pool"]), t(f["v_pool"]), t(f["tables"], torch.int32), t(f["lens"], torch.int32),
            int(f["block_size"]))
    assert rel_err(backend_ref.paged_attention(*args), f["out_full"]) < 2e-6
    assert rel_err(backend_ref.paged_attention(*args, window=12), f["out_w12"]) < 2e-6
    gated = backend_ref.gate(backend_ref.paged_attention(*args), t(f["gate"]))
    assert rel_err(gated, f["out_gated"]) < 2e-6


@pytest.mark.parametrize("bs", [1, 4, 16])
def test_paged_gather_is_the_address_map(bs):
    g = torch.Generator().manual_seed(bs)
    pool = torch.randn(40, bs, 2, 8, generator=g)
    table = torch.randperm(40, generator=g)[:30].to(torch.int32)
    for n, W in ((1, None), (bs * 3 + 1, None), (bs * 7, 5), (29 * bs, bs + 2)):
        K, _ = backend_ref.paged_gather(pool, pool, table, n, bs, W)
        s0 = max(0, n - W) if W else 0
        want = brute.gather_positions(pool.numpy(), table.numpy(), s0, n, bs)
        assert np.array_equal(K.numpy(), want)


def test_paged_equals_contiguous_exactly():
    g = torch.Generator().manual_seed(7)
    lens, bs = [1, 7, 16, 33, 300], 16
    nbs = [-(-n // bs) for n in lens]
    perm = torch.randperm(32, generator=g).tolist()
    rows, at = [], 0
    for n in nbs:
        rows.append(perm[at:at + n] + [0] * (max(nbs) - n))
        at += n
    tables = torch.tensor(rows, dtype=torch.int32)
    kp, vp = torch.randn(32, bs, 2, 64, generator=g), torch.randn(32, bs, 2, 64, generator=g)
    q = torch.randn(5, 8, 64, generator=g)
    got = backend_ref.paged_attention(q, kp, vp, tables, torch.tensor(lens, dtype=torch.int32), bs)
    for i, n in enumerate(lens):
        K = kp[tables[i, :nbs[i]].long()].flatten(0, 1)[:n]
        V = vp[tables[i, :nbs[i]].long()].flatten(0, 1)[:n]
        assert torch.equal(got[i:i + 1], ops_ref.attention(q[i:i + 1], K, V))


# ---------------------------------------------------------------- DeltaNet pieces (ops.py:115-193)

def test_conv_fixture_and_library_conv1d():
    f = np.load(GOLD / "conv.npz")
    out, tail = ops_ref.causal_conv1d(t(f["x"]), t(f["tail"]), t(f["w"]))
    assert rel_err(out, f["out"]) < 1e-6
    assert np.array_equal(tail.numpy(), f["tail_new"].astype(np.float32))
    b_out, b_tail = brute.conv_silu(f["x"], f["tail"], f["w"])
    assert rel_err(out, b_out) < 1e-6


def test_backend_conv_widens_bf16_input_before_the_tail():
    """TorchBackend.causal_conv1d (torch_ref.py:49-50) widens x to fp32 before ops.causal_conv1d, so a bf16 x meets
    the fp32 tail as stored (not rounded to bf16) and the new tail is fp32. Pinned against float64 on the widened
    inputs; a tail rounded to bf16 first (ops.causal_conv1d on the bf16 x as given) must miss that bar."""
    g_ = torch.Generator().manual_seed(41)
    T, C, K = 5, 96, 4
    x = torch.randn(T, C, generator=g_).to(torch.bfloat16)
    tail = torch.randn(K - 1, C, generator=g_)                  # fp32 values that bf16 cannot hold
    assert not torch.equal(tail.to(torch.bfloat16).float(), tail)
    w = 0.5 * torch.randn(C, K, generator=g_)
    u, new_tail = backend_ref.causal_conv1d(x, tail, w)
    b_out, _ = brute.conv_silu(x.double().numpy(), tail.double().numpy(), w.double().numpy())
    assert u.dtype == torch.float32 and new_tail.dtype == torch.float32
    assert rel_err(u, b_out) < 1e-6
    assert torch.equal(new_tail, torch.cat([tail, x.float()])[-(K - 1):])
    # T < K - 1: the carried old rows keep their fp32 bits
    _, short = backend_ref.causal_conv1d(x[:1], tail, w)
    assert torch.equal(short, torch.cat([tail[1:], x[:1].float()]))
    u_rounded, _ = ops_ref.causal_conv1d(x, tail, w)            # the unwidened call rounds the tail to bf16
    assert rel_err(u_rounded.float(), b_out) > 1e-4


def test_l2norm_is_transformers_l2norm():
    from transformers.models.qwen3_5 import modeling_qwen3_5 as hf
    x = torch.randn(5, 16, 128)
    assert torch.equal(ops_ref.l2norm(x), hf.l2norm(x, dim=-1, eps=1e-6))


def test_rms_norm_gated_closed_form():
    x, z, w = torch.randn(6, 128, dtype=torch.float64), torch.randn(6, 128, dtype=torch.float64), torch.randn(128)
    want = x / torch.sqrt((x * x).mean(-1, keepdim=True) + 1e-6) * w.double() * z * torch.sigmoid(z)
    assert rel_err(ops_ref.rms_norm_gated(x.float(), z.float(), w, 1e-6), want) < 1e-6


def delta_inputs():
    f = np.load(GOLD / "delta_rule.npz")
    return f, [t(f[k]) for k in ("q", "k", "v", "beta", "g", "S0")]


def test_recurrent_matches_brute_and_transformers():
    f, (q, k, v, beta, g, S0) = delta_inputs()
    o, S = ops_ref.gated_delta_recurrent(q, k, v, beta, g, S0)
    assert rel_err(o, f["out_brute"]) < 1e-5 and rel_err(S, f["S_brute"]) < 1e-5
    assert rel_err(o, f["out_hf_recurrent"]) < 1e-5 and rel_err(S, f["S_hf_recurrent"]) < 1e-5


def test_chunked_matches_brute_and_transformers():
    f, (q, k, v, beta, g, S0) = delta_inputs()
    o, S = ops_ref.gated_delta_chunked(q, k, v, beta, g, S0)
    assert rel_err(o, f["out_brute"]) < 1e-5 and rel_err(S, f["S_brute"]) < 1e-5
    assert rel_err(o, f["out_hf_chunked"]) < 1e-5 and rel_err(S, f["S_hf_chunked"]) < 1e-5


def test_chunked_matches_brute_at_kernel_shape():
    """dk = dv = 128 with bf16-representable inputs (the fixture the GPU kernel is also checked against)."""
    f = np.load(GOLD / "delta_rule_128.npz")
    wide = lambda b: torch.from_numpy((b.astype(np.uint32) << 16).view(np.float32))
    o, S = ops_ref.gated_delta_chunked(wide(f["q_bf16"]), wide(f["k_bf16"]), wide(f["v_bf16"]), t(f["beta"]),
                                       t(f["g"]), wide(f["S0_bf16"]))
    assert rel_err(o, f["out"]) < 1e-5 and rel_err(S, f["S"]) < 1e-5


@pytest.mark.parametrize("T", [1, 63, 64, 65, 130])
def test_chunked_equals_recurrent(T):
    g_ = torch.Generator().manual_seed(T)
    H, dk, dv = 3, 16, 12
    q = ops_ref.l2norm(torch.randn(T, H, dk, generator=g_)) / dk ** 0.5
    k = ops_ref.l2norm(torch.randn(T, H, dk, generator=g_))
    v = torch.randn(T, H, dv, generator=g_)
    beta = torch.sigmoid(torch.randn(T, H, generator=g_))
    g = -torch.nn.functional.softplus(torch.randn(T, H, generator=g_))
    S0 = torch.randn(H, dk, dv, generator=g_) * 0.1
    o_r, S_r = ops_ref.gated_delta_recurrent(q, k, v, beta, g, S0)
    o_c, S_c = ops_ref.gated_delta_chunked(q, k, v, beta, g, S0)
    assert rel_err(o_c, o_r) < 1e-5 and rel_err(S_c, S_r) < 1e-5


def test_zero_beta_and_decay_leave_state_unchanged():
    T, H, dk, dv = 70, 2, 8, 8
    S0 = torch.randn(H, dk, dv)
    o, S = ops_ref.gated_delta_chunked(torch.randn(T, H, dk), torch.randn(T, H, dk), torch.randn(T, H, dv),
                                       torch.zeros(T, H), torch.zeros(T, H), S0)
    assert torch.allclose(S, S0, rtol=0, atol=1e-6)


def test_deltanet_step_fixture():
    f = np.load(GOLD / "deltanet_step.npz")
    H, dk, dv, key_dim = (int(x) for x in f["dims"])
    st = SlotState(t(f["S"])[None].clone(), t(f["tail"])[None].clone())
    out = backend_ref.deltanet_decode(t(f["qkv"]), t(f["z"]), t(f["b"]), t(f["a"]), st, 0, t(f["conv_w"]),
                                      t(f["A_log"]), t(f["dt_bias"]), t(f["norm_w"]), 1e-6, (H, dk, dv, key_dim))
    assert rel_err(out, f["out"]) < 1e-5
    assert rel_err(st.S[0], f["S_new"]) < 1e-5
    assert np.array_equal(st.conv_tail[0].numpy(), f["tail_new"].astype(np.float32))


def test_softplus_threshold_is_torch_softplus():
    ab = torch.tensor([-30.0, -1.0, 0.0, 5.0, 19.99, 20.0, 20.01, 50.0])
    mine = torch.where(ab > 20, ab, torch.log1p(torch.exp(ab)))
    assert torch.allclose(mine, torch.nn.functional.softplus(ab), rtol=1e-6, atol=0)


# ---------------------------------------------------------------- DeltaNet prefill segment (qwen3_5.py:136-162)

def _dn_layer(seed, H=2, dk=8, dv=8, K=4):
    g_ = torch.Generator().manual_seed(seed)
    C = 2 * H * dk + H * dv
    r = lambda *s, scale=1.0: scale * torch.randn(*s, generator=g_)
    return dict(conv_w=r(C, K, scale=0.5), A_log=r(H, scale=0.5), dt_bias=r(H, scale=0.5),
                norm_w=1.0 + r(dv, scale=0.1), eps=1e-6, dims=(H, dk, dv, H * dk)), C, g_


def test_prefill_segment_equals_chained_decode_steps():
    """One T-token prefill (chunked delta rule, conv over [tail; x], tail handoff) must equal T decode steps (the
    recurrent path pinned by the deltanet_step fixture) token by token: outputs, final S and conv tail."""
    layer, C, g_ = _dn_layer(11)
    H, dk, dv, _ = layer["dims"]
    T = 9
    qkv, z = torch.randn(T, C, generator=g_), torch.randn(T, H * dv, generator=g_)
    b, a = torch.randn(T, H, generator=g_), torch.randn(T, H, generator=g_)
    S0, tail0 = 0.05 * torch.randn(1, H, dk, dv, generator=g_), torch.randn(1, 3, C, generator=g_)
    pre = SlotState(S0.clone(), tail0.clone())
    out = backend_ref.linear_attention_segments(qkv, z, b, a, [pre], 0, [0, T], **layer)
    step = SlotState(S0.clone(), tail0.clone())
    outs = [backend_ref.deltanet_decode(qkv[i:i + 1], z[i:i + 1], b[i:i + 1], a[i:i + 1], step, 0, **layer)
            for i in range(T)]
    assert rel_err(out, torch.cat(outs)) < 1e-5
    assert rel_err(pre.S, step.S) < 1e-5
    assert torch.equal(pre.conv_tail, step.conv_tail)


@pytest.mark.parametrize("split", [1, 2, 5])
def test_prefill_split_in_two_equals_one_prefill(split):
    """A segment prefilled in two pieces (state and conv tail carried) equals the same tokens in one piece; a short
    second piece (fewer tokens than the conv's K - 1) keeps part of the old tail."""
    layer, C, g_ = _dn_layer(12)
    H, dk, dv, _ = layer["dims"]
    T = 7
    qkv, z = torch.randn(T, C, generator=g_), torch.randn(T, H * dv, generator=g_)
    b, a = torch.randn(T, H, generator=g_), torch.randn(T, H, generator=g_)
    S0, tail0 = 0.05 * torch.randn(1, H, dk, dv, generator=g_), torch.randn(1, 3, C, generator=g_)
    one = SlotState(S0.clone(), tail0.clone())
    o1 = backend_ref.linear_attention_segments(qkv, z, b, a, [one], 0, [0, T], **layer)
    two = SlotState(S0.clone(), tail0.clone())
    o2 = torch.cat([backend_ref.linear_attention_segments(qkv[lo:hi], z[lo:hi], b[lo:hi], a[lo:hi], [two], 0,
                                                          [0, hi - lo], **layer)
                    for lo, hi in ((0, split), (split, T))])
    assert rel_err(o2, o1) < 1e-5 and rel_err(two.S, one.S) < 1e-5
    assert torch.equal(two.conv_tail, one.conv_tail)
    assert torch.equal(one.conv_tail[0], qkv[T - 3:])           # the new tail is the last K - 1 raw inputs


def test_prefill_tail_shorter_than_kernel():
    """T = 2 < K - 1 = 3: the new tail is [old tail row 2; x0; x1], the conv of token 0 reads tail rows 0-2."""
    layer, C, g_ = _dn_layer(13)
    H, dk, dv, key_dim = layer["dims"]
    qkv, tail = torch.randn(2, C, generator=g_), torch.randn(3, C, generator=g_)
    q, k, v, beta, g, new_tail = backend_ref.linear_attention_front(qkv, torch.zeros(2, H), torch.zeros(2, H), tail,
                                                                    layer["conv_w"], layer["A_log"],
                                                                    layer["dt_bias"], layer["dims"])
    assert torch.equal(new_tail, torch.cat([tail[2:], qkv]))
    w = layer["conv_w"].double()
    y0 = (tail[0].double() * w[:, 0] + tail[1].double() * w[:, 1] + tail[2].double() * w[:, 2]
          + qkv[0].double() * w[:, 3])
    u0 = y0 / (1 + torch.exp(-y0))
    assert rel_err(v[0].reshape(-1), u0[2 * key_dim:]) < 1e-6
    qn = u0[:key_dim].reshape(H, dk)
    assert rel_err(q[0], qn / qn.norm(dim=-1, keepdim=True) / dk ** 0.5) < 1e-5
    assert torch.allclose(beta, torch.full_like(beta, 0.5))


# ---------------------------------------------------------------- q/k norm + partial RoPE (qwen3_5.py:251-259)

def test_rms_norm_is_transformers_qwen35_rmsnorm():
    """ops.rms_norm with the (1 + w) weight == transformers' Qwen3_5RMSNorm (x * rsqrt(...) * (1 + w)) to rounding."""
    from transformers.models.qwen3_5 import modeling_qwen3_5 as hf
    g_ = torch.Generator().manual_seed(31)
    x, w = torch.randn(7, 3, 256, generator=g_) * 3, 0.1 * torch.randn(256, generator=g_)
    norm = hf.Qwen3_5RMSNorm(256, eps=1e-6)
    with torch.no_grad():
        norm.weight.copy_(w)
        want = norm(x)
    assert rel_err(ops_ref.rms_norm(x, 1.0 + w, 1e-6), want) < 1e-6


def test_rope_is_transformers_apply_rotary_pos_emb():
    """Partial RoPE over the first 64 of 256 dims, theta 1e7: the oracle's rope on the rotated slice equals
    transformers' apply_rotary_pos_emb with cos / sin of the same angles (inv_freq as transformers computes it)."""
    from transformers.models.qwen3_5 import modeling_qwen3_5 as hf
    g_ = torch.Generator().manual_seed(32)
    T, Hq, Hkv, d, rot, theta = 9, 8, 2, 256, 64, 1e7
    q, k = torch.randn(T, Hq, d, generator=g_), torch.randn(T, Hkv, d, generator=g_)
    pos = torch.tensor([0, 1, 2, 100, 4095, 4096, 16383, 20000, 123457], dtype=torch.int32)
    inv = 1.0 / (theta ** (torch.arange(0, rot, 2, dtype=torch.float) / rot))
    assert torch.equal(inv, ops_ref.rope_inv_freq(theta, rot))
    emb = torch.cat([pos.float()[:, None] * inv[None], pos.float()[:, None] * inv[None]], dim=-1)
    hq, hk = hf.apply_rotary_pos_emb(q.transpose(0, 1), k.transpose(0, 1), emb.cos(), emb.sin(), unsqueeze_dim=0)
    qk = ops_ref.rope(torch.cat([q[..., :rot], k[..., :rot]], dim=1), pos, theta)
    assert torch.equal(qk[:, :Hq], hq.transpose(0, 1)[..., :rot])
    assert torch.equal(qk[:, Hq:], hk.transpose(0, 1)[..., :rot])


def test_rope_invariants():
    """Position 0 is the identity; every pair keeps its length; rotating by p then by s equals rotating by p + s
    (to the rounding of the angles); a float64 rotation of the same fp32 angles agrees."""
    g_ = torch.Generator().manual_seed(33)
    x = torch.randn(4, 3, 64, generator=g_)
    zero = torch.zeros(4, dtype=torch.int32)
    assert torch.equal(ops_ref.rope(x, zero, 1e7), x)
    pos = torch.tensor([1, 7, 300, 5000], dtype=torch.int32)
    y = ops_ref.rope(x, pos, 1e7)
    pair = lambda t: t[..., :32] ** 2 + t[..., 32:] ** 2
    assert torch.allclose(pair(y), pair(x), rtol=1e-5, atol=1e-6)
    yy = ops_ref.rope(ops_ref.rope(x, pos, 1e7), pos, 1e7)
    assert rel_err(yy, ops_ref.rope(x, 2 * pos, 1e7)) < 1e-4
    ang = (pos.float()[:, None] * ops_ref.rope_inv_freq(1e7, 64)[None]).double()[:, None, :]
    a, b = x[..., :32].double(), x[..., 32:].double()
    want = torch.cat([a * ang.cos() - b * ang.sin(), a * ang.sin() + b * ang.cos()], dim=-1)
    assert rel_err(y, want) < 1e-6


def test_attention_prep_splits_norms_and_rotates():
    """The composition of qwen3_5.py:251-259 on a small layer: v and the gate are untouched slices, dims past `rot`
    are only normalised, and the rotated q / k heads equal rope(rms_norm(...)) head by head."""
    g_ = torch.Generator().manual_seed(34)
    N, Hq, Hkv, d, rot = 5, 4, 2, 32, 8
    y = torch.randn(N, (2 * Hq + 2 * Hkv) * d, generator=g_)
    qw, kw = 1 + 0.1 * torch.randn(d, generator=g_), 1 + 0.1 * torch.randn(d, generator=g_)
    pos = torch.tensor([0, 3, 9, 27, 81], dtype=torch.int32)
    q, k, v, gate = backend_ref.attention_prep(y, qw, kw, 1e-6, pos, 1e4, rot, (Hq, Hkv, d))
    assert torch.equal(v, y[:, (Hq + Hkv) * d:(Hq + 2 * Hkv) * d].reshape(N, Hkv, d))
    assert torch.equal(gate, y[:, (Hq + 2 * Hkv) * d:])
    qn = ops_ref.rms_norm(y[:, :Hq * d].reshape(N, Hq, d), qw, 1e-6)
    assert torch.equal(q[..., rot:], qn[..., rot:])
    assert torch.equal(q[..., :rot], ops_ref.rope(qn[..., :rot], pos, 1e4))
    kn = ops_ref.rms_norm(y[:, Hq * d:(Hq + Hkv) * d].reshape(N, Hkv, d), kw, 1e-6)
    assert torch.equal(k[..., :rot], ops_ref.rope(kn[..., :rot], pos, 1e4))


# ---------------------------------------------------------------- the rest of a decode step (src/ops.py:18-24, 107-110)

def test_layer_norm_is_the_library_layer_norm():
    """ops.layer_norm (no bias) == torch's layer_norm with that weight, to rounding; with weight 1 every row has mean
    0 and variance 1 (up to eps) -- a dropped centering or a missing eps fails one of them."""
    g_ = torch.Generator().manual_seed(41)
    x, w = torch.randn(6, 2048, generator=g_) * 3 + 1.5, torch.randn(2048, generator=g_)
    want = torch.nn.functional.layer_norm(x, (2048,), w, None, 1e-5)
    assert rel_err(ops_ref.layer_norm(x, w, 1e-5), want) < 1e-6
    y = ops_ref.layer_norm(x.double(), torch.ones(2048, dtype=torch.float64), 0.0)
    assert y.mean(-1).abs().max() < 1e-6 and (y.var(-1, unbiased=False) - 1).abs().max() < 1e-5


def test_silu_mul_is_the_library_silu():
    """silu_mul == torch's silu(g) * u; silu(0) = 0, silu(g) -> g for large g, -> 0 for very negative g."""
    g_ = torch.Generator().manual_seed(42)
    g, u = torch.randn(5, 300, generator=g_) * 4, torch.randn(5, 300, generator=g_)
    assert rel_err(ops_ref.silu_mul(g, u), torch.nn.functional.silu(g) * u) < 1e-6
    edge = torch.tensor([0.0, 30.0, -30.0, -100.0])
    out = ops_ref.silu_mul(edge, torch.ones(4))
    assert out[0] == 0 and abs(out[1] - 30.0) < 1e-6 and abs(out[2]) < 1e-11 and out[3] == 0
