"""Sliding-window decode through ring tables (the second caller of the decode boundary: Cohere2 / Tiny Aya,
src/models/cohere2.py:237-274, whose sliding layers keep each sequence's blocks in a ring, src/state.py:196-359):
histories written block by block through the HIP scatter into rings that wrap several times, each ring slot
NaN-poisoned when it takes a new block, unit 0 (the table's entry for every block below the window) NaN; then one
decode step -- the new token's write and paged_attention(window=W) -- against the oracle's attention over exactly
each window's positions (the values as stored: bf16). Bars: the decode output within 1e-5 relative; the windows
gathered back through the ring tables bit-exact.
"""
import pytest
import torch

import workloads as wl
from helpers import rel_err
from native import kernels
from oracle import ops_ref

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def write_through_rings(k, v, rings, ring, hist, lens, bs, upto):
    """Positions 0 .. upto(n)-1 of every sequence, in order, into ring slot (p // bs) % ring, poisoning a unit
    before its first row of a new block."""
    for units, (K, V), n in zip(rings, hist, lens):
        end = upto(n)
        for b0 in range(0, end, bs):
            u = units[(b0 // bs) % ring]
            k[u], v[u] = float("nan"), float("nan")
            rows = torch.arange(b0, min(end, b0 + bs))
            slots = (u * bs + rows % bs).to(DEV)
            kernels.kv_write(k, v, slots, K[rows].to(DEV), V[rows].to(DEV))


@pytest.mark.parametrize("W,bs,Hq,Hkv,d", [(4096, 16, 16, 4, 128), (100, 16, 8, 2, 256), (37, 4, 8, 2, 64)])
def test_windowed_decode_through_rings(backend, W, bs, Hq, Hkv, d):
    lens = [1, 17, W - 1, W, W + 1, 2 * W + 5, 3 * W + 33] if W < 1000 else [1, 300, 4095, 4096, 4097, 9000, 12001]
    chunk = 512 if W >= 1000 else 16
    gen = torch.Generator().manual_seed(W)
    ring = wl.ring_size(W, bs, chunk)
    tables, units, rings = wl.ring_tables(lens, W, bs, ring, gen)
    k, v = wl.kv_pool((units, bs, Hkv, d), DEV, torch.bfloat16)
    k.fill_(float("nan"))
    v.fill_(float("nan"))
    hist = [(torch.randn(n, Hkv, d, generator=gen), torch.randn(n, Hkv, d, generator=gen)) for n in lens]
    write_through_rings(k, v, rings, ring, hist, lens, bs, lambda n: n - 1)          # the history
    # the decode step: the new token at position n - 1 (its block's ring slot poisoned first when it starts one)
    for units_i, n in zip(rings, lens):
        if (n - 1) % bs == 0:
            u = units_i[((n - 1) // bs) % ring]
            k[u], v[u] = float("nan"), float("nan")
    slots = torch.tensor([units_i[((n - 1) // bs) % ring] * bs + (n - 1) % bs for units_i, n in zip(rings, lens)])
    k_new = torch.stack([K[-1] for K, _ in hist]).to(DEV)
    v_new = torch.stack([V[-1] for _, V in hist]).to(DEV)
    kernels.kv_write(k, v, slots.to(DEV), k_new, v_new)
    q = torch.randn(len(lens), Hq, d, generator=gen)
    lens_t = torch.tensor(lens, dtype=torch.int32, device=DEV)
    out = backend.paged_attention(q.to(DEV), k, v, tables.to(DEV), lens_t, bs, window=W)
    torch.cuda.synchronize()
    assert torch.isfinite(out).all()
    stored = [(K.to(torch.bfloat16).float(), V.to(torch.bfloat16).float()) for K, V in hist]
    want = torch.cat([ops_ref.attention(q[i:i + 1], K[max(0, n - W):], V[max(0, n - W):])
                      for i, ((K, V), n) in enumerate(zip(stored, lens))])
    e = rel_err(out, want)
    print(f"windowed decode W {W} bs {bs} {Hq}/{Hkv} x {d}: rel {e:.2e}")
    assert e < 1e-5
    # the window of every sequence, gathered back through its ring table (HIP gather), is exactly what was stored
    for i, ((K, V), n) in enumerate(zip(stored, lens)):
        lo = max(0, n - W)
        Kg, Vg = kernels.kv_gather(k, v, tables[i].to(DEV), lo, n)
        assert torch.equal(Kg.float().cpu(), K[lo:]) and torch.equal(Vg.float().cpu(), V[lo:])
