"""Backend.attention with T > 1 (src/backend/base.py:32-35; ops.attention, src/ops.py:65-104) and the windowed packed
prefill, both on the prefill attention kernels (rk_paged_prefill), against the CPU oracle.

* attention(q, k, v, causal=True[, window]) on a contiguous cache: T in {2, 63, 64, 65, 512, 2048} over prefixes
  including 0, fp32 and bf16 caches, 8/2 x 256 (Qwen3.5) and 16/4 x 128 (Tiny Aya); group sizes 1, 2, 3, 7 (the
  reference's own 14/2 x 64 kernel-test shape, tests/test_kernels.py:107-114) and 8, head_dim 64 / 128 / 256;
  windows 1 .. 4096 with every key before the first query's window NaN-poisoned; causal=False; a cache longer
  than 65,535 positions read in place.
* The reference's own per-segment prefill sequence (src/models/qwen3_5.py:112-120: kv.write -> kv.read ->
  attention(causal) -> * sigmoid(gate)) on its fp32 pool, driven through RocmBackend's kv scatter / gather and
  attention, equals the packed entry point bit for bit (before the gate) and the oracle within 1e-5.
* paged_prefill_attention(window=W): the sliding layers' prefill (src/models/cohere2.py:155-163) with every pool
  block below each segment's first window NaN-poisoned, bf16 and fp32 pools.

Bars (relative error max|diff| / max|ref| against the fp32 oracle, the reference's convention). The reference
computes in fp32 on widened inputs (src/ops.py:84-87), so every call with an fp32 q or an fp32 cache, and every
exact=True call, runs on fp32 operands and is held to the fp32 bar, 1e-5. q, k and v all bf16 run on bf16 MFMA
operands (probabilities rounded to bf16; 32 queries per wave at 4 query heads per kv-head and head_dim 128 / 256,
16 queries per wave otherwise) and are held to the bf16 bar, 1e-2.
"""
import pytest
import torch

import workloads as wl
from helpers import rel_err
from native import kernels
from oracle import ops_ref, prefill_ref

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
TOL_F32 = 1e-5
TOL_BF16 = 1e-2


def qkv(T, S, Hq, Hkv, d, dtype, seed, qdtype=torch.float32):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(T, Hq, d, generator=g).to(qdtype)
    k = torch.randn(S, Hkv, d, generator=g).to(dtype)
    v = torch.randn(S, Hkv, d, generator=g).to(dtype)
    return q, k, v


def check(backend, q, k, v, tol, label, **kw):
    got = backend.attention(q.to(DEV), k.to(DEV), v.to(DEV), **kw)
    want = ops_ref.attention(q, k, v, **kw)          # widens q, k, v to fp32 as the reference does
    torch.cuda.synchronize()
    e = rel_err(got, want)
    print(f"attention {label}: rel {e:.2e} (bar {tol:g})")
    assert got.shape == q.shape and got.dtype == torch.float32
    assert torch.isfinite(got).all() and e < tol
    return got


@pytest.mark.parametrize("T,P", [(2, 0), (2, 300), (63, 0), (64, 64), (65, 1000), (512, 0), (512, 777), (2048, 0),
                                 (2048, 1000)])
@pytest.mark.parametrize("qdtype,dtype,tol", [(torch.float32, torch.float32, TOL_F32),
                                              (torch.float32, torch.bfloat16, TOL_F32),
                                              (torch.bfloat16, torch.bfloat16, TOL_BF16)])
def test_causal_attention_qwen_heads(backend, T, P, qdtype, dtype, tol):
    q, k, v = qkv(T, T + P, 8, 2, 256, dtype, seed=T * 7 + P, qdtype=qdtype)
    check(backend, q, k, v, tol, f"8/2x256 T {T} prefix {P} q {qdtype} kv {dtype}", causal=True)


@pytest.mark.parametrize("T,P", [(2, 5), (65, 0), (300, 4000), (3, 70000)])
def test_causal_attention_aya_heads(backend, T, P):
    """fp32 q over a bf16 cache (fp32 operands: the cache widened exactly); (3, 70000) reads a cache longer than
    65,535 positions in place."""
    q, k, v = qkv(T, T + P, 16, 4, 128, torch.bfloat16, seed=T + P)
    check(backend, q, k, v, TOL_F32, f"16/4x128 T {T} prefix {P}")


@pytest.mark.parametrize("S", [70003, 70016])
@pytest.mark.parametrize("qdtype,dtype,tol", [(torch.bfloat16, torch.bfloat16, TOL_BF16),
                                              (torch.float32, torch.float32, TOL_F32)])
def test_long_cache_read_in_place(backend, S, qdtype, dtype, tol):
    """Caches past 65,535 positions are viewed in place as blocks of the largest power of two <= 16 dividing S
    (70,003: blocks of one position, a table too long for the kernels' LDS cache, on the 16-query kernels; 70,016:
    blocks of 16)."""
    q, k, v = qkv(65, S, 8, 2, 256, dtype, seed=S, qdtype=qdtype)
    check(backend, q, k, v, tol, f"long cache S {S} q {qdtype} kv {dtype}")


@pytest.mark.parametrize("Hq,Hkv,d", [(14, 2, 64), (8, 8, 128), (16, 8, 64), (12, 4, 256), (16, 2, 128),
                                      (8, 1, 64), (32, 4, 128)])
@pytest.mark.parametrize("dtype,exact,tol", [(torch.float32, False, TOL_F32), (torch.bfloat16, True, TOL_F32),
                                             (torch.bfloat16, False, TOL_BF16)])
@pytest.mark.parametrize("T,P", [(65, 0), (300, 517)])
def test_group_sizes_and_head_dims(backend, Hq, Hkv, d, dtype, exact, tol, T, P):
    """Every group size (14/2 x 64 is the reference's own kernel-test shape) and head_dim 64 / 128 / 256: q, k and v
    in one dtype; fp32, and bf16 with exact=True (widened exactly), on fp32 operands held to 1e-5; bf16 on the
    16-query bf16 kernel held to 1e-2."""
    q, k, v = qkv(T, T + P, Hq, Hkv, d, dtype, seed=Hq * 100 + Hkv * 10 + T, qdtype=dtype)
    got = kernels.attention(q.to(DEV), k.to(DEV), v.to(DEV), exact=exact)
    want = ops_ref.attention(q, k, v)
    e = rel_err(got, want)
    print(f"attention {Hq}/{Hkv}x{d} {dtype} exact {exact} T {T} prefix {P}: rel {e:.2e} (bar {tol:g})")
    assert got.shape == q.shape and torch.isfinite(got).all() and e < tol


@pytest.mark.parametrize("W,T,P", [(16, 65, 600), (16, 2048, 100), (4096, 65, 5000), (4096, 2048, 4200),
                                   (37, 200, 0), (1, 64, 10)])
@pytest.mark.parametrize("qdtype,dtype,tol", [(torch.float32, torch.bfloat16, TOL_F32),
                                              (torch.float32, torch.float32, TOL_F32),
                                              (torch.bfloat16, torch.bfloat16, TOL_BF16)])
def test_windowed_attention_skips_poisoned_history(backend, W, T, P, qdtype, dtype, tol):
    S = T + P
    q, k, v = qkv(T, S, 16, 4, 128, dtype, seed=W + T, qdtype=qdtype)
    cut = max(0, S - T - W + 1)                       # keys before the first query's window: never seen
    k[:cut], v[:cut] = float("nan"), float("nan")
    check(backend, q, k, v, tol, f"window {W} T {T} prefix {P} q {qdtype} kv {dtype}", causal=True, window=W)


@pytest.mark.parametrize("qdtype,dtype,tol", [(torch.float32, torch.float32, TOL_F32),
                                              (torch.bfloat16, torch.bfloat16, TOL_BF16)])
@pytest.mark.parametrize("T,S", [(64, 200), (2, 700), (513, 513)])
def test_non_causal_attention(backend, qdtype, dtype, tol, T, S):
    q, k, v = qkv(T, S, 8, 2, 256, dtype, seed=3 + T, qdtype=qdtype)
    check(backend, q, k, v, tol, f"non-causal T {T} S {S} q {qdtype}", causal=False)


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
    with pytest.raises(NotImplementedError):          # no instance for head_dim 96
        backend.attention(torch.randn(4, 8, 96, device=DEV), torch.randn(4, 2, 96, device=DEV),
                          torch.randn(4, 2, 96, device=DEV))
    with pytest.raises(ValueError):                   # 6 query heads do not split over 4 kv-heads
        backend.attention(torch.randn(4, 6, 128, device=DEV), torch.randn(4, 4, 128, device=DEV),
                          torch.randn(4, 4, 128, device=DEV))
    with pytest.raises(ValueError):                   # more queries than keys
        backend.attention(torch.randn(5, 8, 128, device=DEV), torch.randn(4, 2, 128, device=DEV),
                          torch.randn(4, 2, 128, device=DEV))


def test_exact_request_on_bf16_inputs(backend):
    """bf16 q, k and v at the bf16 kernel's shape: exact=True runs the fp32-operand kernel and meets the fp32 bar;
    the default meets the bf16 bar."""
    q, k, v = qkv(300, 1300, 8, 2, 256, torch.bfloat16, seed=77, qdtype=torch.bfloat16)
    want = ops_ref.attention(q, k, v)
    exact = kernels.attention(q.to(DEV), k.to(DEV), v.to(DEV), exact=True)
    fast = kernels.attention(q.to(DEV), k.to(DEV), v.to(DEV))
    e_exact, e_fast = rel_err(exact, want), rel_err(fast, want)
    print(f"bf16 inputs: exact rel {e_exact:.2e}, bf16 operands rel {e_fast:.2e}")
    assert e_exact < TOL_F32 and e_fast < TOL_BF16


def test_reference_prefill_sequence_through_the_backend(backend):
    """The per-segment loop of Qwen35Model.full_attention (src/models/qwen3_5.py:112-120) with its fp32 pool, run
    as written on RocmBackend (scatter, gather, attention per segment, then the gate in torch), equals the packed
    entry point (P4) bit for bit before the gate, and the oracle within the fp32 bar after it."""
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
    e = rel_err(gated, want.reshape(N, -1))
    print(f"reference prefill sequence, fp32 pool: rel {e:.2e}")
    assert e < TOL_F32


@pytest.mark.parametrize("W", [16, 100, 4096])
@pytest.mark.parametrize("dtype,tol", [(torch.bfloat16, TOL_BF16), (torch.float32, TOL_F32)])
def test_windowed_paged_prefill_with_poisoned_history(backend, W, dtype, tol):
    lengths, starts = [70, 129, 3, 600], [5000, 0, 130, 4200]
    case = wl.prefill_case(lengths, starts, 16, 4, 128, 16, dtype, seed=W)
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
    print(f"windowed paged prefill W {W} {dtype}: rel {e:.2e}")
    assert e < tol
    assert torch.equal(kd.cpu().float().nan_to_num(3.0), kp.float().nan_to_num(3.0))   # the write-back
