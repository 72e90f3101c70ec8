"""Sliding-window decode through the grouped pool (the second caller of the decode boundary: Cohere2 / Tiny Aya,
src/models/cohere2.py:237-274; GroupedKVPool / WindowedSequence, src/state.py:195-359): histories written through
WindowedSequence.write (the HIP scatter) into NaN-poisoned rings that wrap several times, then one decode step —
batch_layout, write_batch, paged_attention(window=W) — against the oracle's attention over exactly each window's
positions (the values as stored: bf16). Bars: the decode output within 1e-5 relative; gathered windows bit-exact.
"""
import pytest
import torch

from helpers import rel_err
from oracle import ops_ref
from state import GroupedKVPool

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def build(W, bs, lens, Hkv, d, chunk, dtype=torch.bfloat16, seed=0):
    pool = GroupedKVPool([W, None], Hkv, d, num_blocks=4096, block_size=bs, max_chunk=chunk, device=DEV,
                         dtype=dtype, poison=True)
    gen = torch.Generator().manual_seed(seed)
    seqs, hist = [pool.new_sequence() for _ in lens], []
    for s, n in zip(seqs, lens):
        K, V = torch.randn(n, Hkv, d, generator=gen), torch.randn(n, Hkv, d, generator=gen)
        for t in range(0, n - 1, chunk):
            e = min(n - 1, t + chunk)
            s.check_forward(t, e)
            s.write(0, t, K[t:e].to(DEV), V[t:e].to(DEV))
            s.advance(e - t)
        hist.append((K.to(dtype).float(), V.to(dtype).float()))
    return pool, seqs, hist, gen


@pytest.mark.parametrize("W,bs,Hq,Hkv,d", [(4096, 16, 16, 4, 128), (100, 16, 8, 2, 256), (37, 4, 8, 2, 64)])
def test_windowed_decode_through_rings(backend, W, bs, Hq, Hkv, d):
    lens = [1, 17, W - 1, W, W + 1, 2 * W + 5, 3 * W + 33] if W < 1000 else [1, 300, 4095, 4096, 4097, 9000, 12001]
    chunk = 512 if W >= 1000 else 16
    pool, seqs, hist, gen = build(W, bs, lens, Hkv, d, chunk)
    g, slot = pool.layer_map[0]
    starts = [n - 1 for n in lens]
    for s, p in zip(seqs, starts):
        s.reserve(p + 1)
    blocks, offsets, tables, lens_t = pool.batch_layout(seqs, starts)
    k_new = torch.stack([K[-1] for K, _ in hist]).to(DEV)
    v_new = torch.stack([V[-1] for _, V in hist]).to(DEV)
    pool.write_batch(slot, blocks[g], offsets, k_new, v_new)
    q = torch.randn(len(lens), Hq, d, generator=gen)
    out = backend.paged_attention(q.to(DEV), pool.k[slot], pool.v[slot], tables[g], lens_t, bs, window=W)
    torch.cuda.synchronize()
    assert torch.isfinite(out).all()
    want = torch.cat([ops_ref.attention(q[i:i + 1], K[max(0, n - W):], V[max(0, n - W):])
                      for i, ((K, V), n) in enumerate(zip(hist, lens))])
    e = rel_err(out, want)
    print(f"windowed decode W {W} bs {bs} {Hq}/{Hkv} x {d}: rel {e:.2e}")
    assert e < 1e-5
    # the gathered window of every sequence (HIP gather through the ring) is exactly what was stored
    for s, (K, V), n in zip(seqs, hist, lens):
        s.advance(1)
        lo = max(0, n - W)
        Kg, Vg = s.read(0, n, lo)
        assert torch.equal(Kg.float().cpu(), K[lo:]) and torch.equal(Vg.float().cpu(), V[lo:])
