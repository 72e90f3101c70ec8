"""Pins of the oracle's two compositions, which restate a sequence of reference calls rather than one function:

* prefill_ref.packed_prefill (src/models/qwen3_5.py:112-120 per segment: kv.write -> kv.read -> attention(causal) ->
  gate; src/state.py:163-180; the 512-query chunking of the reference's prefill) against float64 brute force built
  from the definitions: new rows written by the closed-form address map pool[table[s // bs], s % bs], positions
  0 .. p+n-1 gathered back by the same map, float64 attention with query i at absolute position p + i, and the
  gate as o / (1 + e^-gate). Segments cover n > 512 (the chunk loop's second chunk sees keys up to p + c1 - 1), a
  start inside a partially filled block, an empty prefix, a one-token segment, fp32 and bf16 pools.
* decode_ref.hybrid_decode_step (src/models/qwen3_5.py:228-290) against a float64 composition written here from the
  model's definitions (numpy loops, brute.attention and brute.deltanet_step), on a tiny 4-layer stack.

CPU only."""
import math

import numpy as np
import pytest
import torch

import workloads as wl
from helpers import rel_err
from oracle import brute, decode_ref, prefill_ref


def _pool_prefill_case(pool_dtype, bs, segs, seed=7, Hq=8, Hkv=2, d=16):
    """segs: [(prefix p, new n)]. A pool of random blocks with each segment's table a slice of a seeded permutation
    (non-contiguous blocks); the prefix rows hold N(0,1) values, unused rows NaN (never read)."""
    g = torch.Generator().manual_seed(seed)
    need = [-(-(p + n) // bs) for p, n in segs]
    NB = sum(need) + 5
    perm = torch.randperm(NB, generator=g)
    max_nb = max(need)
    tables = torch.zeros(len(segs), max_nb, dtype=torch.int32)
    o = 0
    for s, nb in enumerate(need):
        tables[s, :nb] = perm[o:o + nb].int()
        o += nb
    k_pool = torch.full((NB, bs, Hkv, d), float("nan"))
    v_pool = torch.full((NB, bs, Hkv, d), float("nan"))
    for s, (p, n) in enumerate(segs):
        for pos in range(p):
            blk, r = int(tables[s, pos // bs]), pos % bs
            k_pool[blk, r] = torch.randn(Hkv, d, generator=g)
            v_pool[blk, r] = torch.randn(Hkv, d, generator=g)
    k_pool, v_pool = k_pool.to(pool_dtype), v_pool.to(pool_dtype)
    N = sum(n for _, n in segs)
    q = torch.randn(N, Hq, d, generator=g)
    k_new, v_new = torch.randn(N, Hkv, d, generator=g), torch.randn(N, Hkv, d, generator=g)
    gate = torch.randn(N, Hq * d, generator=g)
    cu = [0]
    for _, n in segs:
        cu.append(cu[-1] + n)
    return q, k_new, v_new, k_pool, v_pool, tables, cu, [p for p, _ in segs], gate


@pytest.mark.parametrize("pool_dtype,bs,segs", [
    (torch.float32, 4, [(0, 600), (5, 37), (130, 1), (9, 70)]),     # n > 512; start inside block 1; one token
    (torch.bfloat16, 16, [(33, 530), (0, 3), (16, 16)]),             # bf16 pool rounds the written rows
])
def test_packed_prefill_matches_brute_force(pool_dtype, bs, segs):
    q, k_new, v_new, k_pool, v_pool, tables, cu, starts, gate = _pool_prefill_case(pool_dtype, bs, segs)
    kp_ref, vp_ref = k_pool.float().numpy().copy(), v_pool.float().numpy().copy()
    kp, vp = k_pool.clone(), v_pool.clone()
    got = prefill_ref.packed_prefill(q, k_new, v_new, kp, vp, tables, cu, starts, bs, gate)

    # brute force: write by the address map (values rounded to the pool type, as the pool stores them)
    kn = k_new.to(pool_dtype).float().numpy()
    vn = v_new.to(pool_dtype).float().numpy()
    want = np.zeros((cu[-1],) + tuple(q.shape[1:]))
    for s, p in enumerate(starts):
        lo, hi = cu[s], cu[s + 1]
        tab = tables[s].numpy()
        for i in range(hi - lo):
            pos = p + i
            kp_ref[tab[pos // bs], pos % bs] = kn[lo + i]
            vp_ref[tab[pos // bs], pos % bs] = vn[lo + i]
        K = brute.gather_positions(kp_ref, tab, 0, p + hi - lo, bs)
        V = brute.gather_positions(vp_ref, tab, 0, p + hi - lo, bs)
        want[lo:hi] = brute.attention(q[lo:hi].numpy(), K, V, causal=True)   # query i at (p + n) - n + i = p + i
    gd = gate.double().numpy().reshape(want.shape)
    want = want / (1.0 + np.exp(-gd))

    assert rel_err(got, want) < 2e-6
    # the written pool is the address map's, bit for bit (NaN rows untouched)
    assert np.array_equal(kp.float().numpy(), kp_ref, equal_nan=True)
    assert np.array_equal(vp.float().numpy(), vp_ref, equal_nan=True)


def test_packed_prefill_chunk_boundary_keys():
    """Query 512 (the first of the second chunk) must see keys up to its own position and no further: perturbing
    the key one past it leaves its output unchanged, perturbing its own key changes it."""
    q, k_new, v_new, k_pool, v_pool, tables, cu, starts, _ = _pool_prefill_case(torch.float32, 4, [(6, 520)])
    base = prefill_ref.packed_prefill(q, k_new, v_new, k_pool.clone(), v_pool.clone(), tables, cu, starts, 4)
    k2 = k_new.clone()
    k2[513] += 5.0
    after = prefill_ref.packed_prefill(q, k2, v_new, k_pool.clone(), v_pool.clone(), tables, cu, starts, 4)
    assert torch.equal(base[:513], after[:513]) and not torch.equal(base[513], after[513])


# ---------------------------------------------------------------- the decode step composition

TINY = wl.HybridConfig(layers=4, hidden=32, intermediate=48, vocab=50, Hq=4, Hkv=1, d=16, rot=8, theta=1e4,
                       H=2, dk=8, dv=8, block_size=4)


def _rms64(x, w, eps):
    return x / np.sqrt((x * x).mean(-1, keepdims=True) + eps) * w


def _rope64(x, positions, theta, rot):
    """rotate_half pairs (i, i + rot/2) over the first rot dims, float64 angles position / theta^(i / (rot/2))."""
    x = x.copy()
    half = rot // 2
    for t, pos in enumerate(positions):
        for i in range(half):
            ang = pos / theta ** (i / half)
            c, s = math.cos(ang), math.sin(ang)
            a, b = x[t, :, i].copy(), x[t, :, i + half].copy()
            x[t, :, i], x[t, :, i + half] = a * c - b * s, a * s + b * c
    return x


def _decode64(cfg, w, k_pool, v_pool, S, conv, seq_rows, slot, tables, lens, tokens):
    """float64 decode step of the hybrid stack, from the model's definitions (src/models/qwen3_5.py:228-290)."""
    W = {n: t.double().numpy() for n, t in w.items()}
    B = len(tokens)
    h = W["embed_tokens.weight"][tokens]
    for i in range(cfg.layers):
        p = f"layers.{i}."
        x = _rms64(h, W[p + "input_layernorm.weight"], cfg.eps)
        L = slot[i]
        if cfg.is_full(i):
            a = p + "self_attn."
            Hq, Hkv, d = cfg.Hq, cfg.Hkv, cfg.d
            y = x @ W[a + "qkvg.weight"].T
            q = _rms64(y[:, :Hq * d].reshape(B, Hq, d), W[a + "q_norm.weight"], cfg.eps)
            k = _rms64(y[:, Hq * d:(Hq + Hkv) * d].reshape(B, Hkv, d), W[a + "k_norm.weight"], cfg.eps)
            v = y[:, (Hq + Hkv) * d:(Hq + 2 * Hkv) * d].reshape(B, Hkv, d)
            gate = y[:, (Hq + 2 * Hkv) * d:]
            pos = [int(n) - 1 for n in lens]
            q, k = _rope64(q, pos, cfg.theta, cfg.rot), _rope64(k, pos, cfg.theta, cfg.rot)
            o = np.zeros((B, Hq, d))
            for j in range(B):
                tab = tables[j].numpy()
                blk, r = tab[pos[j] // cfg.block_size], pos[j] % cfg.block_size
                k_pool[L][blk, r], v_pool[L][blk, r] = k[j], v[j]
                K = brute.gather_positions(k_pool[L], tab, 0, pos[j] + 1, cfg.block_size)
                V = brute.gather_positions(v_pool[L], tab, 0, pos[j] + 1, cfg.block_size)
                o[j] = brute.attention(q[j:j + 1], K, V)[0]
            o = o.reshape(B, Hq * d) / (1.0 + np.exp(-gate))
            h = h + o @ W[a + "o_proj.weight"].T
        else:
            a = p + "linear_attn."
            C, Z, H = cfg.conv_dim, cfg.H * cfg.dv, cfg.H
            y = x @ W[a + "in_proj.weight"].T
            o = np.zeros((B, Z))
            for j, r in enumerate(seq_rows):
                o[j], conv[r, L], S[r, L] = brute.deltanet_step(
                    y[j:j + 1, :C], y[j, C:C + Z], y[j, C + Z:C + Z + H], y[j, C + Z + H:], conv[r, L], S[r, L],
                    W[a + "conv1d.weight"], W[a + "A_log"], W[a + "dt_bias"], W[a + "norm.weight"], cfg.eps,
                    (H, cfg.dk, cfg.dv, H * cfg.dk))
            h = h + o @ W[a + "out_proj.weight"].T
        x = _rms64(h, W[p + "post_attention_layernorm.weight"], cfg.eps)
        gu = x @ W[p + "mlp.gate_up.weight"].T
        F = gu.shape[1] // 2
        h = h + (gu[:, :F] / (1.0 + np.exp(-gu[:, :F])) * gu[:, F:]) @ W[p + "mlp.down_proj.weight"].T
    return _rms64(h, W["norm.weight"], cfg.eps) @ W["embed_tokens.weight"].T


def test_decode_ref_matches_float64_composition():
    cfg = TINY
    w = wl.hybrid_weights(cfg, seed=5)
    g = torch.Generator().manual_seed(6)
    lens_before = [3, 9, 1]                       # history lengths; the step writes position lens_before[j]
    B = len(lens_before)
    n_full = sum(cfg.is_full(i) for i in range(cfg.layers))
    n_lin = cfg.layers - n_full
    slot, fi, li = [], 0, 0
    for i in range(cfg.layers):
        slot.append(fi if cfg.is_full(i) else li)
        fi, li = fi + cfg.is_full(i), li + (not cfg.is_full(i))
    bs = cfg.block_size
    need = [-(-(n + 1) // bs) for n in lens_before]
    NB = sum(need) + 3
    perm = torch.randperm(NB, generator=g)
    tables = torch.zeros(B, max(need), dtype=torch.int32)
    o = 0
    for j, nb in enumerate(need):
        tables[j, :nb] = perm[o:o + nb].int()
        o += nb
    k_pool = torch.randn(n_full, NB, bs, cfg.Hkv, cfg.d, generator=g)
    v_pool = torch.randn(n_full, NB, bs, cfg.Hkv, cfg.d, generator=g)
    seqs = 5
    S = 0.02 * torch.randn(seqs, n_lin, cfg.H, cfg.dk, cfg.dv, generator=g)
    conv = torch.randn(seqs, n_lin, cfg.conv_k - 1, cfg.conv_dim, generator=g)
    seq_index = torch.tensor([4, 0, 2])
    lens = torch.tensor([n + 1 for n in lens_before], dtype=torch.int32)
    positions = torch.tensor(lens_before, dtype=torch.int32)
    slots = torch.tensor([int(tables[j, p // bs]) * bs + p % bs for j, p in enumerate(lens_before)])
    tokens = torch.tensor([7, 0, 49])

    k64, v64 = k_pool.double().numpy().copy(), v_pool.double().numpy().copy()
    S64, conv64 = S.double().numpy().copy(), conv.double().numpy().copy()
    want = _decode64(cfg, w, k64, v64, S64, conv64, seq_index.tolist(), slot, tables, lens, tokens.numpy())

    kp, vp, Sr, cr = k_pool.clone(), v_pool.clone(), S.clone(), conv.clone()
    got = decode_ref.hybrid_decode_step(cfg, w, kp, vp, Sr, cr, seq_index, slot, slots, tables, lens, positions,
                                        tokens)
    assert rel_err(got, want) < 1e-5
    assert rel_err(Sr, S64) < 1e-5 and rel_err(cr, conv64) < 1e-6
    assert rel_err(kp, k64) < 1e-5 and rel_err(vp, v64) < 1e-5
    untouched = [r for r in range(seqs) if r not in seq_index.tolist()]
    assert torch.equal(Sr[untouched], S[untouched]) and torch.equal(cr[untouched], conv[untouched])
