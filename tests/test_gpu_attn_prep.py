"""Parity of rk_attn_prep — the per-head q / k RMSNorm (1 + w), partial RoPE and decode KV write of a gated-attention
layer (src/models/qwen3_5.py:251-262; :100-110 for prefill) — with the CPU oracle (ops.rms_norm, ops.rope and their
composition in oracle/backend_ref.attention_prep, pinned against transformers' Qwen3.5 RMSNorm and
apply_rotary_pos_emb), and of the whole decode attention layer built on it (prep + paged decode + fused gate).

Bars: q, k (fp32) within 1e-5 relative; v is a copy (bit-exact in an fp32 pool, and rounded exactly as torch's
.to(torch.bfloat16) in a bf16 pool); a bf16 pool's k rows within the bf16 bar 1e-2 of the oracle's fp32 k (and equal
to the oracle's k rounded to bf16 except where the fp32 values differ in the last bits at a rounding boundary); pool
rows outside the slots untouched.
"""
import pytest
import torch

from helpers import rel_err
from oracle import backend_ref

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
TOL = 1e-5


def layer(seed, N, Hq, Hkv, d, dtype=torch.float32):
    g_ = torch.Generator().manual_seed(seed)
    y = torch.randn(N, (2 * Hq + 2 * Hkv) * d, generator=g_) * 2
    qw, kw = 1 + 0.1 * torch.randn(d, generator=g_), 1 + 0.1 * torch.randn(d, generator=g_)
    return y.to(dtype), qw, kw, g_


@pytest.mark.parametrize("d,rot", [(256, 64), (128, 32), (64, 64), (256, 0), (256, 256)])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_prefill_mode_matches_oracle(backend, d, rot, dtype):
    N, Hq, Hkv, theta = 300, 8, 2, 1e7
    y, qw, kw, g_ = layer(d + rot, N, Hq, Hkv, d, dtype)
    pos = torch.randint(0, 20000, (N,), generator=g_, dtype=torch.int32)
    q_ref, k_ref, v_ref, gate_ref = backend_ref.attention_prep(y, qw, kw, 1e-6, pos, theta, rot, (Hq, Hkv, d))
    q, k, v, gate = backend.attention_prep(y.to(DEV), qw.to(DEV), kw.to(DEV), 1e-6, pos.to(DEV), theta, rot,
                                           (Hq, Hkv, d))
    eq, ek = rel_err(q, q_ref), rel_err(k, k_ref)
    print(f"prep d {d} rot {rot} {dtype}: q rel {eq:.2e}, k rel {ek:.2e}")
    assert eq < TOL and ek < TOL
    assert torch.equal(v.cpu(), v_ref)
    assert torch.equal(gate.cpu(), gate_ref)


def _pool_case(seed, pool_dtype, B=64, Hq=8, Hkv=2, d=256, nb=256, bs=16):
    y, qw, kw, g_ = layer(seed, B, Hq, Hkv, d)
    k_pool = torch.randn(nb, bs, Hkv, d, generator=g_).to(pool_dtype)
    v_pool = torch.randn(nb, bs, Hkv, d, generator=g_).to(pool_dtype)
    slots = torch.randperm(nb * bs, generator=g_)[:B].to(torch.int64)
    pos = torch.randint(0, 16384, (B,), generator=g_, dtype=torch.int32)
    return y, qw, kw, k_pool, v_pool, slots, pos


@pytest.mark.parametrize("pool_dtype", [torch.float32, torch.bfloat16])
def test_decode_mode_writes_the_pool(backend, pool_dtype):
    Hq, Hkv, d, rot, theta = 8, 2, 256, 64, 1e7
    y, qw, kw, k_pool, v_pool, slots, pos = _pool_case(7, pool_dtype)
    q_ref, k_ref, v_ref, _ = backend_ref.attention_prep(y, qw, kw, 1e-6, pos, theta, rot, (Hq, Hkv, d))
    kp, vp = k_pool.to(DEV), v_pool.to(DEV)
    q, gate = backend.attention_prep(y.to(DEV), qw.to(DEV), kw.to(DEV), 1e-6, pos.to(DEV), theta, rot, (Hq, Hkv, d),
                                     kp, vp, slots.to(DEV))
    assert rel_err(q, q_ref) < TOL
    bs = k_pool.shape[1]
    got_k = kp.cpu().view(-1, Hkv, d)[slots]
    got_v = vp.cpu().view(-1, Hkv, d)[slots]
    assert torch.equal(got_v, v_ref.to(pool_dtype))                 # write_batch: v.to(pool dtype)
    if pool_dtype == torch.float32:
        assert rel_err(got_k, k_ref) < TOL
    else:
        assert rel_err(got_k.float(), k_ref) < 1e-2
        same = (got_k == k_ref.to(pool_dtype)).float().mean().item()
        print(f"bf16 k rows equal to the oracle's rounding: {same:.5f}")
        assert same > 0.999
    rest = torch.ones(k_pool.shape[0] * bs, dtype=torch.bool)
    rest[slots] = False
    assert torch.equal(kp.cpu().view(-1, Hkv, d)[rest], k_pool.view(-1, Hkv, d)[rest])
    assert torch.equal(vp.cpu().view(-1, Hkv, d)[rest], v_pool.view(-1, Hkv, d)[rest])


def test_out_of_range_slot_is_skipped(backend):
    Hq, Hkv, d = 8, 2, 256
    y, qw, kw, k_pool, v_pool, slots, pos = _pool_case(8, torch.bfloat16, B=4, nb=8)
    slots[1] = 8 * 16                                                 # one past the pool
    slots[2] = -1
    kp, vp = k_pool.to(DEV), v_pool.to(DEV)
    backend.attention_prep(y.to(DEV), qw.to(DEV), kw.to(DEV), 1e-6, pos.to(DEV), 1e7, 64, (Hq, Hkv, d), kp, vp,
                           slots.to(DEV))
    changed = (kp.cpu() != k_pool).view(-1, Hkv * d).any(dim=1).nonzero().flatten().tolist()
    assert changed == sorted([int(slots[0]), int(slots[3])])


def test_decode_attention_layer_end_to_end(backend):
    """prep (norms, RoPE, KV write) + paged decode with the fused gate == the reference's decode steps
    (qwen3_5.py:251-271: norms, rope, write_batch, paged_attention, * sigmoid(gate)) on a bf16 pool."""
    from oracle import backend_ref as br
    import workloads as wl
    Hq, Hkv, d, rot, theta, B, bs = 8, 2, 256, 64, 1e7, 16, 16
    g_ = torch.Generator().manual_seed(9)
    lens = torch.randint(1, 200, (B,), generator=g_).tolist()
    tables = wl.scattered_tables(lens, 128, bs, g_)
    kh, vh = wl.kv_pool((1, 128, bs, Hkv, d), "cpu", torch.bfloat16)
    for i, n in enumerate(lens):                                     # history of n - 1 tokens, then the new one
        for p in range(n - 1):
            kh[0, int(tables[i, p // bs]), p % bs] = torch.randn(Hkv, d, generator=g_).to(torch.bfloat16)
            vh[0, int(tables[i, p // bs]), p % bs] = torch.randn(Hkv, d, generator=g_).to(torch.bfloat16)
    starts = [n - 1 for n in lens]
    blocks = torch.tensor([int(tables[i, p // bs]) for i, p in enumerate(starts)])
    offsets = torch.tensor([p % bs for p in starts])
    lens_t = torch.tensor(lens, dtype=torch.int32)
    y, qw, kw, _ = layer(10, B, Hq, Hkv, d)
    pos = torch.tensor(starts, dtype=torch.int32)
    # oracle on CPU copies of the pool
    k_ref_pool, v_ref_pool = kh[0].clone(), vh[0].clone()
    q_ref, k_ref, v_ref, gate = br.attention_prep(y, qw, kw, 1e-6, pos, theta, rot, (Hq, Hkv, d))
    k_ref_pool[blocks, offsets] = k_ref.to(torch.bfloat16)
    v_ref_pool[blocks, offsets] = v_ref.to(torch.bfloat16)
    o_ref = br.gate(br.paged_attention(q_ref, k_ref_pool, v_ref_pool, tables, lens_t, bs).reshape(B, Hq * d), gate)
    # device
    kp, vp = kh[0].to(DEV), vh[0].to(DEV)
    slots = (blocks * bs + offsets).to(DEV)
    q, g_dev = backend.attention_prep(y.to(DEV), qw.to(DEV), kw.to(DEV), 1e-6, pos.to(DEV), theta, rot,
                                      (Hq, Hkv, d), kp, vp, slots)
    assert g_dev.stride(0) == y.shape[1]                            # the gate columns of y, read in place
    o = backend.paged_attention(q, kp, vp, tables.to(DEV), lens_t.to(DEV), bs, gate=g_dev)
    e = rel_err(o.reshape(B, Hq * d), o_ref)
    print(f"decode attention layer: rel {e:.2e}")
    assert e < 1e-2                                                   # bf16 pool: k rows may round differently
    o2 = backend.paged_attention(q, kp, vp, tables.to(DEV), lens_t.to(DEV), bs, gate=g_dev.contiguous())
    assert torch.equal(o, o2)                                         # strided gate rows == a contiguous copy
