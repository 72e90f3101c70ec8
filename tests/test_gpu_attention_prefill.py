"""Backend.attention with T > 1 (src/backend/base.py:32-35; ops.attention, src/ops.py:65-104) and the windowed packed
prefill, both on the prefill attention kernel (rk_paged_prefill), against the CPU oracle.

* attention(q, k, v, causal=True[, window]) on a contiguous cache: T in {2, 63, 64, 65, 512, 2048} over prefixes
  including 0, fp32 and bf16 caches, 8/2 x 256 (Qwen3.5) and 16/4 x 128 (Tiny Aya); windows 16 and 4096 with every
  key before the first query's window NaN-poisoned; causal=False.
* The reference's own per-segment prefill sequence (src/models/qwen3_5.py:112-120: kv.write -> kv.read ->
  attention(causal) -> * sigmoid(gate)), driven through RocmBackend's kv scatter / gather and attention, equals the
  packed entry point bit for bit (before the gate) and the oracle within the bar.
* paged_prefill_attention(window=W): the sliding layers' prefill (src/models/cohere2.py:155-163) with every pool
  block below each segment's first window NaN-poisoned.

The products run on bf16 MFMA operands (q, k, v rounded to bf16 as staged; probabilities rounded) with fp32
accumulation: outputs are held to the bf16 bar, 1e-2 relative (max|diff| / max|ref|) of the fp32 oracle."""
import pytest
import torch

import workloads as wl
from helpers import rel_err
from native import kernels
from oracle import ops_ref, prefill_ref

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
TOL = 1e-2


def qkv(T, S, Hq, Hkv, d, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(T, Hq, d, generator=g)
    k = torch.randn(S, Hkv, d, generator=g).to(dtype)
    v = torch.randn(S, Hkv, d, generator=g).to(dtype)
    return q, k, v


@pytest.mark.parametrize("T,P", [(2, 0), (2, 300), (63, 0), (64, 64), (65, 1000), (512, 0), (512, 777), (2048, 0),
                                 (2048, 1000)])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_causal_attention_qwen_heads(backend, T, P, dtype):
    q, k, v = qkv(T, T + P, 8, 2, 256, dtype, seed=T * 7 + P)
    got = backend.attention(q.to(DEV), k.to(DEV), v.to(DEV), causal=True)
    want = ops_ref.attention(q, k.float(), v.float(), causal=True)
    torch.cuda.synchronize()
    e = rel_err(got, want)
    print(f"attention T {T} prefix {P} {dtype}: rel {e:.2e}")
    assert got.shape == (T, 8, 256) and got.dtype == torch.float32
    assert torch.isfinite(got).all() and e < TOL


@pytest.mark.parametrize("T,P", [(2, 5), (65, 0), (300, 4000), (3, 70000)])
def test_causal_attention_aya_heads(backend, T, P):
    q, k, v = qkv(T, T + P, 16, 4, 128, torch.bfloat16, seed=T + P)
    got = backend.attention(q.to(DEV), k.to(DEV), v.to(DEV))
    assert rel_err(got, ops_ref.attention(q, k.float(), v.float())) < TOL


@pytest.mark.parametrize("W,T,P", [(16, 65, 600), (16, 2048, 100), (4096, 65, 5000), (4096, 2048, 4200),
                                   (37, 200, 0), (1, 64, 10)])
def test_windowed_attention_skips_poisoned_history(backend, W, T, P):
    S = T + P
    q, k, v = qkv(T, S, 16, 4, 128, torch.bfloat16, seed=W + T)
    cut = max(0, S - T - W + 1)                       # keys before the first query's window: never seen
    k[:cut], v[:cut] = float("nan"), float("nan")
    got = backend.attention(q.to(DEV), k.to(DEV), v.to(DEV), causal=True, window=W)
    want = ops_ref.attention(q, k.float(), v.float(), causal=True, window=W)
    torch.cuda.synchronize()
    assert torch.isfinite(got).all()
    e = rel_err(got, want)
    print(f"windowed attention W {W} T {T} prefix {P}: rel {e:.2e}")
    assert e < TOL


def test_non_causal_attention(backend):
    q, k, v = qkv(64, 200, 8, 2, 256, torch.float32, seed=3)
    got = backend.attention(q.to(DEV), k.to(DEV), v.to(DEV), causal=False)
    assert rel_err(got, ops_ref.attention(q, k, v, causal=False)) < TOL


def test_strided_views_and_refusals(backend):
    """k / v as column slices of a projection output (the model's state-None branch passes k[sg.lo:sg.hi] of a
    reshaped view) give the same result as contiguous copies; unsupported shapes raise."""
    g = torch.Generator().manual_seed(4)
    y = torch.randn(70, (8 + 2 + 2) * 256, generator=g).to(DEV)
    q = y[:, :8 * 256].reshape(70, 8, 256)
    k = y[:, 8 * 256:10 * 256].reshape(70, 2, 256)
    v = y[:, 10 * 256:].reshape(70, 2, 256)
    a = backend.attention(q, k, v)
    b = backend.attention(q.contiguous(), k.contiguous(), v.contiguous())
    assert torch.equal(a, b)
    with pytest.raises(NotImplementedError):
        backend.attention(torch.randn(4, 8, 64, device=DEV), torch.randn(4, 2, 64, device=DEV),
                          torch.randn(4, 2, 64, device=DEV))
    with pytest.raises(ValueError):
        backend.attention(torch.randn(5, 8, 128, device=DEV), torch.randn(4, 2, 128, device=DEV),
                          torch.randn(4, 2, 128, device=DEV))


def test_reference_prefill_sequence_through_the_backend(backend):
    """The per-segment loop of Qwen35Model.full_attention (src/models/qwen3_5.py:112-120) with its fp32 pool, run
    as written on RocmBackend (scatter, gather, attention per segment, then the gate in torch), equals the packed
    entry point (P4) bit for bit before the gate, and the oracle within the bar after it."""
    case = wl.prefill_case([70, 129, 3, 40], [50, 0, 500, 16], 8, 2, 256, 16, torch.float32, seed=12)
    c = case.to(DEV)
    bs = c.block_size
    kp, vp = c.k_pool.clone(), c.v_pool.clone()
    outs = []
    for s in range(len(c.starts)):
        lo, hi, p = c.cu_seqlens[s], c.cu_seqlens[s + 1], c.starts[s]
        table = c.tables[s]
        pos = torch.arange(p, p + hi - lo, device=DEV)
        slots = table[pos // bs].long() * bs + pos % bs
        kernels.kv_write(kp, vp, slots, c.k_new[lo:hi], c.v_new[lo:hi])            # kv.write(slot, start, k, v)
        ks, vs = kernels.kv_gather(kp, vp, table, 0, p + hi - lo)                 # kv.read(slot, start + T)
        outs.append(backend.attention(c.q[lo:hi], ks, vs, causal=True))           # b.attention(qs, ks, vs)
    o = torch.cat(outs)
    packed_pool_k, packed_pool_v = c.k_pool.clone(), c.v_pool.clone()
    packed = backend.paged_prefill_attention(c.q, c.k_new, c.v_new, packed_pool_k, packed_pool_v, c.tables,
                                             c.cu_seqlens, c.starts, bs)
    torch.cuda.synchronize()
    assert torch.equal(o, packed)
    assert torch.equal(kp, packed_pool_k) and torch.equal(vp, packed_pool_v)
    N = o.shape[0]
    gated = o.reshape(N, -1) * torch.sigmoid(c.gate)                              # o * sigmoid(gate)
    ref = case.clone()
    want = prefill_ref.packed_prefill(ref.q, ref.k_new, ref.v_new, ref.k_pool, ref.v_pool, ref.tables,
                                      ref.cu_seqlens, ref.starts, bs, ref.gate)
    assert rel_err(gated, want.reshape(N, -1)) < TOL


@pytest.mark.parametrize("W", [16, 100, 4096])
def test_windowed_paged_prefill_with_poisoned_history(backend, W):
    lengths, starts = [70, 129, 3, 600], [5000, 0, 130, 4200]
    case = wl.prefill_case(lengths, starts, 16, 4, 128, 16, torch.bfloat16, seed=W)
    bs = case.block_size
    kp, vp = case.k_pool.clone(), case.v_pool.clone()
    for s, p in enumerate(starts):                    # every block below the segment's first window: NaN
        for b in range(max(0, p - W + 1) // bs):
            blk = int(case.tables[s, b])
            kp[blk], vp[blk] = float("nan"), float("nan")
    c = case.to(DEV)
    kd, vd = kp.to(DEV), vp.to(DEV)
    got = backend.paged_prefill_attention(c.q, c.k_new, c.v_new, kd, vd, c.tables, c.cu_seqlens, c.starts, bs,
                                          gate=c.gate, window=W)
    torch.cuda.synchronize()
    assert torch.isfinite(got).all()
    # oracle: the reference's windowed segment loop (src/models/cohere2.py:155-163): write, read from the first
    # query's window, attention(causal, window), then the gate
    outs = []
    for s, p in enumerate(starts):
        lo, hi = case.cu_seqlens[s], case.cu_seqlens[s + 1]
        tab = case.tables[s].long()
        pos = torch.arange(p, p + hi - lo)
        kp[tab[pos // bs], pos % bs] = case.k_new[lo:hi].to(kp.dtype)
        vp[tab[pos // bs], pos % bs] = case.v_new[lo:hi].to(vp.dtype)
        first = max(0, p - W + 1)
        allpos = torch.arange(first, p + hi - lo)
        K, V = kp[tab[allpos // bs], allpos % bs].float(), vp[tab[allpos // bs], allpos % bs].float()
        outs.append(ops_ref.attention(case.q[lo:hi], K, V, causal=True, window=W))
    want = torch.cat(outs)
    want = (want.reshape(want.shape[0], -1) * torch.sigmoid(case.gate.float())).reshape(want.shape)
    e = rel_err(got, want)
    print(f"windowed paged prefill W {W}: rel {e:.2e}")
    assert e < TOL
    assert torch.equal(kd.cpu().float().nan_to_num(3.0), kp.float().nan_to_num(3.0))   # the write-back
