"""P4 parity on seeded random shapes: the packed prefill (rk_paged_prefill) against the oracle over group sizes,
head dims, block sizes, segment lengths and prefixes, windows, gates, dtypes, exact requests and split sizes drawn
from one seeded generator, so that every case runs one of the three kernels (bf16 operands at 32 or 16 queries per
wave, fp32 operands) in combinations the targeted tests do not list.

Expected values: the reference's per-segment write -> read -> attention (causal, with the window when one is drawn)
-> gate (src/models/qwen3_5.py:112-120, src/models/cohere2.py:155-163, src/ops.py:65-104), restated by
oracle/prefill_ref.py and oracle/ops_ref.py. Bars as for the other prefill tests: 1e-2 relative for bf16 operands,
1e-5 for fp32 operands; the pool after the write-back bit-exact.
"""
import pytest
import torch

import workloads as wl
from helpers import rel_err
from native import kernels
from oracle import ops_ref, prefill_ref

DEV = "cuda:0"
TOL = {"bf16_32": 1e-2, "bf16_16": 1e-2, "fp32": 1e-5}
N_CASES = 24


def draw(seed: int) -> dict:
    g = torch.Generator().manual_seed(20_000 + seed)
    pick = lambda xs: xs[int(torch.randint(len(xs), (1,), generator=g))]
    Hkv = pick([1, 2, 4])
    G = pick([1, 2, 3, 4, 4, 5, 7, 8])
    S = int(torch.randint(1, 5, (1,), generator=g))
    return {
        "Hkv": Hkv, "Hq": Hkv * G, "d": pick([64, 128, 256]), "bs": pick([1, 4, 16, 16, 32]),
        "lengths": torch.randint(1, 300, (S,), generator=g).tolist(),
        "starts": torch.randint(0, 3000, (S,), generator=g).tolist(),
        "dtype": pick([torch.bfloat16, torch.bfloat16, torch.float32]),
        "exact": pick([False, False, True]), "gate": pick([True, False]),
        "window": pick([None, None, 1, 37, 512]), "split": pick([None, None, 0, 2, 5]),
    }


def expected(case: wl.PrefillCase, window, gate: bool):
    c = case.clone()
    if window is None:
        out = prefill_ref.packed_prefill(c.q, c.k_new, c.v_new, c.k_pool, c.v_pool, c.tables, c.cu_seqlens,
                                         c.starts, c.block_size, c.gate if gate else None)
        return out, c.k_pool, c.v_pool
    bs, outs = c.block_size, []
    for s in range(len(c.starts)):                  # the same write -> read as packed_prefill, then the window
        lo, hi, p = c.cu_seqlens[s], c.cu_seqlens[s + 1], c.starts[s]
        table = c.tables[s].long()
        pos = torch.arange(p, p + hi - lo)
        c.k_pool[table[pos // bs], pos % bs] = c.k_new[lo:hi].to(c.k_pool.dtype)
        c.v_pool[table[pos // bs], pos % bs] = c.v_new[lo:hi].to(c.v_pool.dtype)
        nb = -(-(p + hi - lo) // bs)
        K = c.k_pool[table[:nb]].flatten(0, 1)[:p + hi - lo]
        V = c.v_pool[table[:nb]].flatten(0, 1)[:p + hi - lo]
        outs.append(ops_ref.attention(c.q[lo:hi], K, V, causal=True, window=window))
    out = torch.cat(outs)
    if gate:
        out = (out.reshape(out.shape[0], -1) * torch.sigmoid(c.gate.float())).reshape(out.shape)
    return out, c.k_pool, c.v_pool


@pytest.mark.gpu
@pytest.mark.parametrize("seed", range(N_CASES))
def test_random_prefill(backend, monkeypatch, seed):
    p = draw(seed)
    case = wl.prefill_case(p["lengths"], p["starts"], p["Hq"], p["Hkv"], p["d"], p["bs"], p["dtype"], seed=seed)
    max_nb = case.tables.shape[1]
    which = kernels.prefill_kernel(case.q.dtype, case.k_pool.dtype, p["Hq"], p["Hkv"], p["d"], p["exact"], max_nb,
                                   p["bs"])
    want, wk, wv = expected(case, p["window"], p["gate"])
    monkeypatch.setattr(kernels, "PREFILL_SPLIT_TILES", p["split"])
    c = case.to(DEV)
    got = backend.paged_prefill_attention(c.q, c.k_new, c.v_new, c.k_pool, c.v_pool, c.tables, c.cu_seqlens,
                                          c.starts, c.block_size, gate=c.gate if p["gate"] else None,
                                          window=p["window"], exact=p["exact"])
    torch.cuda.synchronize()
    err = rel_err(got, want)
    print(f"random prefill {seed}: {which} {p['Hq']}/{p['Hkv']}x{p['d']} bs {p['bs']} {p['dtype']} exact "
          f"{p['exact']} window {p['window']} split {p['split']} lengths {p['lengths']} starts {p['starts']}: "
          f"rel err {err:.2e}")
    assert got.shape == case.q.shape and torch.isfinite(got).all() and err < TOL[which]
    assert torch.equal(c.k_pool.cpu(), wk) and torch.equal(c.v_pool.cpu(), wv)


def test_random_cases_reach_every_kernel():
    """The seeded draw covers all three kernels and the window / split / exact options (checked on the CPU)."""
    seen, opts = set(), set()
    for seed in range(N_CASES):
        p = draw(seed)
        nb = max(-(-(n + s) // p["bs"]) for n, s in zip(p["lengths"], p["starts"]))
        seen.add(kernels.prefill_kernel(p["dtype"], p["dtype"], p["Hq"], p["Hkv"], p["d"], p["exact"], nb, p["bs"]))
        opts |= {("window", p["window"] is not None), ("split", p["split"] not in (None, 0)), ("exact", p["exact"])}
    assert seen == {"bf16_32", "bf16_16", "fp32"}
    assert {("window", True), ("split", True), ("exact", True)} <= opts
